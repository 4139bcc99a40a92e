// Optimizer-side kernels over flat parameter arenas: the fused Adam step
// with a device-resident update counter and the sum of squared gradients,
// a standalone sum of squares, the Polyak blend and a fill kernel.
//
// Reference semantics:
//   Adam (S = m/(1-b1), V = v/(1-b2) storage, fused scalars)
//                          ttrl/engine/optim/adam.py:93-134, ttrl/engine/optim/scalars.py:13-27
//   grad_sq_device         ttrl/algos/grads.py:46-60
//   Polyak blend           ttrl/algos/sac/targets.py:45-52
//
// The Adam scalars depend on the update count t.  The count lives on the
// device, so one captured graph replays correctly for every t: the update
// kernel reads t_old and uses t = t_old + 1, and the finishing kernel (one
// block, after every update block has run) stores t and the reduced
// sum of squares.  All reductions are fixed-order.
#include "adam_dev.hpp"
#include "common.hpp"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <mutex>
#include <utility>
#include <vector>

namespace ttrl {

constexpr int kOptThreads = 256;
constexpr int kOptMaxBlocks = 1024;

float* ctx_workspace(ttrl_ctx* ctx, long* floats);

// The update of four consecutive parameters with gradient gv, element by
// element in order (adam1); g^2 is added to gsq in that order.
__device__ __forceinline__ void adam4(f32x4& pv, const f32x4& gv, f32x4& sv, f32x4& vv, float b1, float b2, float wd,
                                      float eps_t, float alpha_t, float& gsq) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    float pq = pv[q], sq = sv[q], vq = vv[q];
    adam1(pq, gv[q], sq, vq, b1, b2, wd, eps_t, alpha_t, gsq);
    pv[q] = pq;
    sv[q] = sq;
    vv[q] = vq;
  }
}

// A gradient scale applied as the step reads g (NoScale: none).
// A step's gradient scale in two halves: issue() starts its loads, finish()
// forms it from them (the step's scalars are formed in between).
struct NoScale {
  static constexpr bool kOn = false;
  struct Loads {};
  __device__ Loads issue() const { return {}; }
  __device__ float finish(const Loads&) const { return 1.f; }
};

// The update of float4s map(j), j = first, first + step, ... below end,
// g^2 added to gsq in that order.  The next float4's loads are in flight
// while one is computed, and the first float4's are issued before the
// step's scalars are formed (thread 0's double-precision powers) and, with
// a Scale, before the gradient scale is formed, so those latencies overlap.
// Every thread of the workgroup calls it (the scalars' barrier); alpha_t and
// eps_t receive the scalars, *gscale the gradient scale.
template <class Map, class Scale = NoScale>
__device__ __forceinline__ void adam_loop(float* __restrict__ p, const float* __restrict__ g, float* __restrict__ S,
                                          float* __restrict__ V, long first, long end, long step,
                                          const int* __restrict__ stepc, float lr, float b1, float b2, float eps,
                                          float wd, float& gsq, float* alpha_t, float* eps_t, Map map,
                                          Scale scale = Scale{}, float* gscale = nullptr) {
  // the update count first, through the scalar cache: thread 0's wait for
  // it then waits for none of the first float4's loads, and the scalars'
  // arithmetic runs while they are in flight
  const int step_now = *(const __attribute__((address_space(1))) int*)stepc;
  f32x4* P = reinterpret_cast<f32x4*>(p);
  const f32x4* G = reinterpret_cast<const f32x4*>(g);
  f32x4* Sv = reinterpret_cast<f32x4*>(S);
  f32x4* Vv = reinterpret_cast<f32x4*>(V);
  long j = first;
  bool have = j < end;
  long i = have ? map(j) : 0;
  f32x4 pv = {}, gv = {}, sv = {}, vv = {};
  if (have) {
    pv = P[i];
    gv = G[i];
    sv = Sv[i];
    vv = Vv[i];
  }
  const typename Scale::Loads sl = scale.issue();
  adam_scalars_of(step_now, lr, b1, b2, eps, alpha_t, eps_t);
  float gs = 1.f;
  if constexpr (Scale::kOn) gs = scale.finish(sl);
  if (gscale) *gscale = gs;
  const float at = *alpha_t, et = *eps_t;
  while (have) {
    const long jn = j + step;
    const bool more = jn < end;
    const long in = more ? map(jn) : 0;
    f32x4 pn = {}, gn = {}, sn = {}, vn = {};
    if (more) {
      pn = P[in];
      gn = G[in];
      sn = Sv[in];
      vn = Vv[in];
    }
    if constexpr (Scale::kOn) {
      gv = gv * gs;
      if (gs != 1.f) const_cast<f32x4*>(G)[i] = gv;  // the clipped gradient, as the clip leaves it
    }
    adam4(pv, gv, sv, vv, b1, b2, wd, et, at, gsq);
    P[i] = pv;
    Sv[i] = sv;
    Vv[i] = vv;
    j = jn;
    i = in;
    have = more;
    pv = pn;
    gv = gn;
    sv = sn;
    vv = vn;
  }
}

struct Identity {
  __device__ long operator()(long j) const { return j; }
};

// Block `blk` of `nblk` of one Adam update: its grid-stride share of the
// range and its partial sum of g^2 into partials[blk].  The same code serves
// a single-range launch and a range of a multi-range launch, so both give
// the same bits.
template <class Scale = NoScale>
__device__ __forceinline__ void adam_block(float* __restrict__ p, const float* __restrict__ g,
                                           float* __restrict__ S, float* __restrict__ V, long n,
                                           const int* __restrict__ step, float lr, float b1, float b2, float eps,
                                           float wd, float* __restrict__ partials, int blk, int nblk,
                                           Scale scale = Scale{}) {
  __shared__ float red[kOptThreads / 64];
  float alpha_t, eps_t, gs;
  float gsq = 0.f;
  const long n4 = n / 4;
  const long stride = long(nblk) * kOptThreads;
  adam_loop(p, g, S, V, blk * long(kOptThreads) + threadIdx.x, n4, stride, step, lr, b1, b2, eps, wd, gsq, &alpha_t,
            &eps_t, Identity{}, scale, &gs);
  // Tail (n % 4) handled by block 0.
  if (blk == 0) {
    for (long i = n4 * 4 + threadIdx.x; i < n; i += kOptThreads) {
#pragma clang fp contract(off)
      float graw = g[i];
      if constexpr (Scale::kOn) {
        graw *= gs;
        if (gs != 1.f) const_cast<float*>(g)[i] = graw;
      }
      gsq += graw * graw;
      const float gg = wd != 0.f ? graw + wd * p[i] : graw;
      V[i] = gg * gg + b2 * V[i];
      S[i] = gg + b1 * S[i];
      p[i] = p[i] - (S[i] / (sqrtf(V[i]) + eps_t)) * alpha_t;
    }
  }
  const float tot = block_sum<kOptThreads>(gsq, red);
  if (threadIdx.x == 0) partials[blk] = tot;
}

__global__ __launch_bounds__(kOptThreads) void k_adam(float* __restrict__ p, const float* __restrict__ g,
                                                      float* __restrict__ S, float* __restrict__ V, long n,
                                                      const int* __restrict__ step, float lr, float b1, float b2,
                                                      float eps, float wd, float* __restrict__ partials) {
  adam_block(p, g, S, V, n, step, lr, b1, b2, eps, wd, partials, int(blockIdx.x), int(gridDim.x));
}

// The global-norm clip's scale (k_clip_scale's) from the sum of g^2 left as
// partial sums: every workgroup adds them as k_finish does, so each forms
// the same sum; workgroup 0 stores it and the norm.
// The norm partials (nparts <= kOptMaxBlocks) are loaded kClipLoads to a
// thread and summed in the order a loop over i = tid, tid + kOptThreads, ...
// adds them.
constexpr int kClipLoads = kOptMaxBlocks / kOptThreads;
static_assert(kOptMaxBlocks % kOptThreads == 0, "whole loads per thread");
struct ClipScale {
  static constexpr bool kOn = true;
  const float* parts;
  int nparts;
  float max_norm;
  float* sq_out;
  float* norm_out;
  struct Loads {
    float v[kClipLoads];
  };
  __device__ Loads issue() const {
    Loads l;
#pragma unroll
    for (int k = 0; k < kClipLoads; ++k) l.v[k] = parts[min(int(threadIdx.x) + k * kOptThreads, nparts - 1)];
    return l;
  }
  __device__ float finish(const Loads& l) const {
    __shared__ float red[kOptThreads / 64];
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < kClipLoads; ++k)
      if (int(threadIdx.x) + k * kOptThreads < nparts) s += l.v[k];
    const float sq = block_sum<kOptThreads>(s, red);
    const double total = std::sqrt(double(sq));
    if (blockIdx.x == 0 && threadIdx.x == 0) {
      if (sq_out) *sq_out = sq;
      if (norm_out) *norm_out = float(total);
    }
    return total > double(max_norm) ? float(double(max_norm) / (total + 1e-6)) : 1.f;
  }
};

// clip_grad_norm and the step in one pass over g: the step reads g times the
// clip's scale and, when that is not 1, writes the clipped g back.
__global__ __launch_bounds__(kOptThreads) void k_adam_clip(float* __restrict__ p, float* __restrict__ g,
                                                           float* __restrict__ S, float* __restrict__ V, long n,
                                                           const int* __restrict__ step, float lr, float b1,
                                                           float b2, float eps, float wd,
                                                           float* __restrict__ partials, ClipScale clip) {
  adam_block(p, g, S, V, n, step, lr, b1, b2, eps, wd, partials, int(blockIdx.x), int(gridDim.x), clip);
}

// Up to kMultiRanges deferred Adam ranges and a Polyak blend in one launch:
// blocks [r.block0, r.block0 + r.blocks) run range r (r.blocks = the grid a
// single-range launch of it uses), the rest the blend.
constexpr int kMultiRanges = 4;
struct AdamRange {
  float* p;
  const float* g;
  float* S;
  float* V;
  long n;
  const int* step;
  float lr, b1, b2, eps, wd;
  float* partials;
  int block0, blocks;
};
struct AdamMulti {
  AdamRange r[kMultiRanges];
  int nr;
  float* pd;
  const float* ps;
  long pn;
  float keep, tau;
  int pblock0, pblocks;
};
__global__ __launch_bounds__(kOptThreads) void k_adam_multi(AdamMulti a) {
  const int b = int(blockIdx.x);
#pragma unroll
  for (int i = 0; i < kMultiRanges; ++i) {
    if (i >= a.nr) break;
    const AdamRange& r = a.r[i];
    if (b >= r.block0 && b < r.block0 + r.blocks) {
      adam_block(r.p, r.g, r.S, r.V, r.n, r.step, r.lr, r.b1, r.b2, r.eps, r.wd, r.partials, b - r.block0,
                 r.blocks);
      return;
    }
  }
  const long stride = long(a.pblocks) * kOptThreads;
  for (long i = (b - a.pblock0) * long(kOptThreads) + threadIdx.x; i < a.pn; i += stride)
    a.pd[i] = a.pd[i] * a.keep + a.ps[i] * a.tau;
}

// The finishes of up to kAdamSlots deferred steps, one block each: the
// partials of slot f.slot[b] summed as k_finish sums them.
struct FinishSlots {
  const float* parts[kAdamSlots];
  int count[kAdamSlots];
  int* step[kAdamSlots];
  float* out[kAdamSlots];
  int accumulate[kAdamSlots];
};
__global__ __launch_bounds__(kOptThreads) void k_finish_slots(FinishSlots f) {
  __shared__ float red[kOptThreads / 64];
  const int b = int(blockIdx.x);
  float s = 0.f;
  for (int i = threadIdx.x; i < f.count[b]; i += kOptThreads) s += f.parts[b][i];
  const float tot = block_sum<kOptThreads>(s, red);
  if (threadIdx.x == 0) {
    if (f.out[b]) *f.out[b] = f.accumulate[b] ? *f.out[b] + tot : tot;
    *f.step[b] = *f.step[b] + 1;
  }
}

__global__ __launch_bounds__(kOptThreads) void k_finish(const float* __restrict__ partials, int nparts,
                                                        int* __restrict__ step, float* __restrict__ out,
                                                        int accumulate) {
  __shared__ float red[kOptThreads / 64];
  float s = 0.f;
  for (int i = threadIdx.x; i < nparts; i += kOptThreads) s += partials[i];
  const float tot = block_sum<kOptThreads>(s, red);
  if (threadIdx.x == 0) {
    if (out) *out = accumulate ? *out + tot : tot;
    if (step) *step = *step + 1;
  }
}

// k_finish that also ends a replayed learner step: the metric ring's row
// ring[c][0..n) = metrics when 0 <= c < slots, c = *counter, then
// *counter = c + 1 (what ttrl_step_end does in a launch of its own).
__global__ __launch_bounds__(kOptThreads) void k_finish_end(const float* __restrict__ partials, int nparts,
                                                            int* __restrict__ step, float* __restrict__ out,
                                                            int accumulate, int* __restrict__ counter,
                                                            const float* __restrict__ metrics, int n,
                                                            float* __restrict__ ring, int slots) {
  __shared__ float red[kOptThreads / 64];
  float s = 0.f;
  for (int i = threadIdx.x; i < nparts; i += kOptThreads) s += partials[i];
  const float tot = block_sum<kOptThreads>(s, red);
  const int c = *counter;
  if (c >= 0 && c < slots)
    for (int i = threadIdx.x; i < n; i += kOptThreads) ring[long(c) * n + i] = metrics[i];
  __syncthreads();
  if (threadIdx.x == 0) {
    if (out) *out = accumulate ? *out + tot : tot;
    if (step) *step = *step + 1;
    *counter = c + 1;
  }
}

// ----------------------------------------------------- gradient sources ---
//
// A source's gradient is formed a float4 at a time: float4 q < nw4 covers
// elements 4q .. 4q+3 of its [rows][cols] weight block, the next nb4 its
// bias (elements past cols are the arena's padding: zero).  Each element is
// summed in the order its unreduced launch would have used, so the step
// writes the same bits that launch's own reduction would have.
constexpr int kMaxGradSources = 8;
constexpr int kMaxOrderedSums = 4;
constexpr int kSplitBatch = 16;  // split partials of a float4 in flight together
constexpr int kOuterBatch = 8;   // batch rows of an outer-product float4 in flight together (general path)
constexpr int kOuterLds = 2048;   // v floats an outer-product source stages in LDS
constexpr int kOuterULds = 6144;  // u floats (the workgroup's slice of rows) it stages
constexpr int kOuterChunk = 32;   // batch rows of u staged per memory round trip
constexpr int kSumLds = 1024;    // terms of an ordered sum staged in LDS
// A wide outer-product source (cols a multiple of kTileCols, batch <=
// kTileBatch) is formed by tiles: one workgroup per kTileRows x kTileCols
// block of the weight, kTileOuts float4s per thread (tile rows tr and
// tr + 16 of one float4 column), its slices of u and v staged in LDS, so
// each workgroup reads [batch][32] of u and [batch][64] of v however wide
// the layer is, and a layer of 3136 x 512 takes 784 workgroups (one wave of
// the chip's resident workgroups with the rest of the step).  The bias's
// gradient (sum_b v[b][c]) is formed by the first row band's tiles, from
// the rows of v they have staged: lanes 0 .. kTileCols/4 - 1 of wave 0 take
// one float4 of the tile's columns each.
constexpr int kTileRows = 32, kTileCols = 64, kTileBatch = 32;
constexpr int kTileBand = kOptThreads / (kTileCols / 4);  // tile rows one pass of the workgroup covers
constexpr int kTileOuts = kTileRows / kTileBand;
static_assert(kTileRows % kTileBand == 0 && kTileOuts == 2, "a tile is two float4s per thread");
static_assert(kTileBatch * kTileRows <= kOuterULds && kTileBatch * kTileCols <= kOuterLds, "a tile's slices fit");

struct GradSrc {
  int kind, rows, cols, splits, batch;
  float scale, bias_scale;
  float* gw;       // where the weight block's gradient is written
  float* gb;       // the bias's (null: none)
  long w4, b4;     // the same places as float4 indexes of the arena (Adam only)
  int nw4, nb4;
  const float* part;
  long sstride;    // floats per split
  const float* u;
  const float* v;
  FDiv dc;         // division by cols
  int block0, blocks;
  int tiled, ntc, ntiles;  // tiled outer product: tiles per row band, tiles (the first band's also form the bias)
};

__device__ __forceinline__ f32x4 source_grad(const GradSrc& s, int q, bool* bias, int* qq) {
  *bias = q >= s.nw4;
  *qq = *bias ? q - s.nw4 : q;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  if (s.kind == TTRL_GRAD_SPLITS) {
    const float* base = s.part + (*bias ? long(s.rows) * s.cols : 0L) + 4L * *qq;
    for (int s0 = 0; s0 < s.splits; s0 += kSplitBatch) {
      f32x4 v[kSplitBatch];
#pragma unroll
      for (int j = 0; j < kSplitBatch; ++j)
        v[j] = *reinterpret_cast<const f32x4*>(base + long(min(s0 + j, s.splits - 1)) * s.sstride);
#pragma unroll
      for (int j = 0; j < kSplitBatch; ++j)
        if (s0 + j < s.splits) {  // uniform
          acc.x += v[j].x;
          acc.y += v[j].y;
          acc.z += v[j].z;
          acc.w += v[j].w;
        }
    }
    // the weight-gradient epilogue's alpha * acc + 0 (bias row: bias_scale)
    const float sc = *bias ? s.bias_scale : s.scale;
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] = fmaf(sc, acc[c], 0.f);
    return acc;
  }
  // outer product: element e of the weight block is (r, c) = divmod(e, cols)
  int r[4], c[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = 4 * *qq + j;
    r[j] = *bias ? 0 : s.dc.div(e);
    c[j] = *bias ? min(e, s.cols - 1) : e - r[j] * s.cols;
  }
  for (int b0 = 0; b0 < s.batch; b0 += kOuterBatch) {
    float uu[kOuterBatch][4], vv[kOuterBatch][4];
#pragma unroll
    for (int i = 0; i < kOuterBatch; ++i) {
      const long bb = min(b0 + i, s.batch - 1);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uu[i][j] = s.u[bb * s.rows + r[j]];
        vv[i][j] = s.v[bb * s.cols + c[j]];
      }
    }
#pragma unroll
    for (int i = 0; i < kOuterBatch; ++i)
      if (b0 + i < s.batch)  // uniform
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = fmaf(*bias ? 1.f : uu[i][j], vv[i][j], acc[j]);
  }
  if (*bias)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = 4 * *qq + j < s.cols ? acc[j] : 0.f;
  return acc;
}

// The rows of u an outer-product source's workgroup reads: its float4s
// [qb0, qb0 + kOptThreads) cover weight elements from 4 qb0 on, rows
// [r_lo, r_lo + R).  The workgroup stages that slice of u ([batch][R]) and
// all of v ([batch][cols]) in LDS when they fit (R <= kOptThreads), one
// memory round trip per kOuterChunk batch rows, and forms its float4s from
// LDS; otherwise (staged false) each thread reads u and v itself.
struct OuterSlice {
  int r_lo, R;
  bool staged;
};
__device__ __forceinline__ OuterSlice outer_slice(const GradSrc& s, int qb0) {
  OuterSlice o{0, 0, false};
  if (s.kind != TTRL_GRAD_OUTER) return o;
  const int qw1 = min(qb0 + kOptThreads, s.nw4);
  if (qw1 > qb0) {
    o.r_lo = s.dc.div(4 * qb0);
    o.R = s.dc.div(4 * qw1 - 1) - o.r_lo + 1;
  }
  o.staged = o.R <= kOptThreads && s.batch * o.R <= kOuterULds && s.batch * s.cols <= kOuterLds;
  return o;
}
__device__ __forceinline__ void stage_outer(const GradSrc& s, const OuterSlice& o, float* us, float* vs) {
  const int tid = threadIdx.x, nv = s.batch * s.cols;
  const int rr = min(tid, max(o.R - 1, 0));
  for (int b0 = 0; b0 < s.batch; b0 += kOuterChunk) {
    float t[kOuterChunk];
#pragma unroll
    for (int i = 0; i < kOuterChunk; ++i) t[i] = s.u[long(min(b0 + i, s.batch - 1)) * s.rows + o.r_lo + rr];
    const float vv = b0 == 0 && tid < nv ? s.v[tid] : 0.f;
    if (b0 == 0 && tid < nv) vs[tid] = vv;
#pragma unroll
    for (int i = 0; i < kOuterChunk; ++i)
      if (tid < o.R && b0 + i < s.batch) us[(b0 + i) * o.R + tid] = t[i];
  }
  for (int i = kOptThreads + tid; i < nv; i += kOptThreads) vs[i] = s.v[i];
  __syncthreads();
}
// stage_outer in two halves when the batch is at most kOuterChunk rows:
// issue_stage loads the thread's rows (every load unconditional: threads
// past the slice repeat its last row or v's last element, and write
// nothing), commit_stage writes them to LDS (with v past kOptThreads
// elements) and waits for the workgroup.
struct StageLoads {
  float u[kOuterChunk];
  float v;
};
__device__ __forceinline__ StageLoads issue_stage(const GradSrc& s, const OuterSlice& o) {
  const int tid = threadIdx.x, nv = s.batch * s.cols;
  const int rr = min(tid, max(o.R - 1, 0));
  StageLoads l;
#pragma unroll
  for (int i = 0; i < kOuterChunk; ++i) l.u[i] = s.u[long(min(i, s.batch - 1)) * s.rows + o.r_lo + rr];
  l.v = s.v[min(tid, nv - 1)];
  return l;
}
__device__ __forceinline__ void commit_stage(const GradSrc& s, const OuterSlice& o, const StageLoads& l, float* us,
                                             float* vs) {
  const int tid = threadIdx.x, nv = s.batch * s.cols;
  if (tid < nv) vs[tid] = l.v;
#pragma unroll
  for (int i = 0; i < kOuterChunk; ++i)
    if (tid < o.R && i < s.batch) us[i * o.R + tid] = l.u[i];
  for (int i = kOptThreads + tid; i < nv; i += kOptThreads) vs[i] = s.v[i];
  __syncthreads();
}
// source_grad of a staged outer-product source: the same sums in the same
// order (b from zero, fmaf(u, v, acc); the bias adds v), read from LDS.
__device__ __forceinline__ f32x4 outer_grad_staged(const GradSrc& s, const OuterSlice& o, const float* us,
                                                   const float* vs, int q, bool* bias, int* qq) {
  *bias = q >= s.nw4;
  *qq = *bias ? q - s.nw4 : q;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  if (*bias) {
    int c[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) c[j] = min(4 * *qq + j, s.cols - 1);
    for (int b = 0; b < s.batch; ++b)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] = fmaf(1.f, vs[b * s.cols + c[j]], acc[j]);
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = 4 * *qq + j < s.cols ? acc[j] : 0.f;
    return acc;
  }
  int r[4], c[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = 4 * *qq + j, rj = s.dc.div(e);
    r[j] = rj - o.r_lo;
    c[j] = e - rj * s.cols;
  }
  for (int b = 0; b < s.batch; ++b)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = fmaf(us[b * o.R + r[j]], vs[b * s.cols + c[j]], acc[j]);
  return acc;
}

// A tile's slices: loaded into registers (issue_outer_tile), then written
// to LDS (commit_outer_tile): us[b][i] = u[b][r0 + i] (rows past the block
// repeat its last row, never used), vs[b][j] = v[b][c0 + j].  Work that does
// not need them can run between the two while the loads are in flight.
struct OuterTileLoads {
  float u[kTileBatch * kTileRows / kOptThreads];
  f32x4 v[kTileBatch * kTileCols / 4 / kOptThreads];
};
__device__ __forceinline__ OuterTileLoads issue_outer_tile(const GradSrc& s, int r0, int c0) {
  constexpr int NU = kTileBatch * kTileRows / kOptThreads, NV = kTileBatch * kTileCols / 4 / kOptThreads;
  const int tid = threadIdx.x;
  OuterTileLoads l;
#pragma unroll
  for (int k = 0; k < NU; ++k) {
    const int e = tid + k * kOptThreads, b = e / kTileRows, i = e - b * kTileRows;
    l.u[k] = b < s.batch ? s.u[long(b) * s.rows + min(r0 + i, s.rows - 1)] : 0.f;
  }
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int e = tid + k * kOptThreads, b = e / (kTileCols / 4), j = e - b * (kTileCols / 4);
    l.v[k] = b < s.batch ? *reinterpret_cast<const f32x4*>(s.v + long(b) * s.cols + c0 + 4 * j) : f32x4{};
  }
  return l;
}
__device__ __forceinline__ void commit_outer_tile(const OuterTileLoads& l, float* us, float* vs) {
  constexpr int NU = kTileBatch * kTileRows / kOptThreads, NV = kTileBatch * kTileCols / 4 / kOptThreads;
  const int tid = threadIdx.x;
#pragma unroll
  for (int k = 0; k < NU; ++k) us[tid + k * kOptThreads] = l.u[k];
#pragma unroll
  for (int k = 0; k < NV; ++k) reinterpret_cast<f32x4*>(vs)[tid + k * kOptThreads] = l.v[k];
  __syncthreads();
}
// The thread's kTileOuts float4s (tile rows tr + kTileBand * o, float4
// column tc4): the same sums in the same order as source_grad (b from zero,
// fmaf(u, v, acc)).  The staged rows past the batch hold zeros, and adding
// fmaf(0, 0, acc) = acc + 0 leaves acc's bits as they are (acc starts at +0
// and a sum rounded to nearest is never -0 unless both terms are), so the
// loop runs over all kTileBatch rows, unrolled by 8 (fully, its hoisted
// reads would not fit the registers).
__device__ __forceinline__ void outer_grad_tile(const float* us, const float* vs, int tr, int tc4,
                                                f32x4 (&acc)[kTileOuts]) {
#pragma unroll
  for (int o = 0; o < kTileOuts; ++o) acc[o] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
  for (int b = 0; b < kTileBatch; ++b) {
    const f32x4 v = reinterpret_cast<const f32x4*>(vs)[b * (kTileCols / 4) + tc4];
#pragma unroll
    for (int o = 0; o < kTileOuts; ++o) {
      const float u = us[b * kTileRows + tr + kTileBand * o];
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[o][j] = fmaf(u, v[j], acc[o][j]);
    }
  }
}
// The bias float4 of the tile's float4 column tc4: sum_b v[b][c] in the
// order source_grad adds it (b from zero; the zero rows past the batch, as
// above, change nothing).
__device__ __forceinline__ f32x4 outer_bias_tile(const float* vs, int tc4) {
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
  for (int b = 0; b < kTileBatch; ++b) {
    const f32x4 v = reinterpret_cast<const f32x4*>(vs)[b * (kTileCols / 4) + tc4];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = fmaf(1.f, v[j], acc[j]);
  }
  return acc;
}
// Where workgroup t of a tiled source works: its tile (the thread's float4
// q[o] of the weight, ok[o] false past the block's rows) and, in the first
// row band of a source with a bias, the bias: bias_wave for wave 0 (uniform
// over the wave), bias_lane for its lanes that step bias float4 qb (the
// tile's float4 column tc4 = tid; the other lanes' qb repeats the last).
// The tile that block blk of a tiled source's blocks [block0, block0 + T)
// forms.  Workgroups go to the chip's eight XCDs in turn (block b to XCD
// b % 8), each XCD with an L2 of its own, and the tiles of one row band
// share their slice of u: the blocks of one XCD take a contiguous run of
// tiles (XCD x the run after the blocks of XCDs 0 .. x-1), so a band's slice
// is fetched into one L2, not eight.  A bijection onto [0, T).
__device__ __forceinline__ int xcd_tile(int blk, int block0, int T) {
  const int x = blk & 7;
  int start = 0;
#pragma unroll
  for (int y = 0; y < 7; ++y)  // blocks of the range on XCD y: (T - offset of its first + 7) / 8
    if (y < x) start += (T - ((y - block0) & 7) + 7) >> 3;
  const int first = block0 + ((x - block0) & 7);
  return start + ((blk - first) >> 3);
}

struct TileSpot {
  int r0, c0, tr, tc4;
  int q[kTileOuts];
  bool ok[kTileOuts];
  bool bias_wave, bias_lane;
  int qb;
};
__device__ __forceinline__ TileSpot tile_spot(const GradSrc& s, int t) {
  const int tid = threadIdx.x;
  TileSpot o{};
  o.tr = tid / (kTileCols / 4);
  o.tc4 = tid % (kTileCols / 4);
  const int band = t / s.ntc;
  o.r0 = band * kTileRows;
  o.c0 = (t - band * s.ntc) * kTileCols;
#pragma unroll
  for (int k = 0; k < kTileOuts; ++k) {
    const int row = o.r0 + o.tr + kTileBand * k;
    o.ok[k] = row < s.rows;
    o.q[k] = int((long(row) * s.cols + o.c0 + 4 * o.tc4) / 4);
  }
  o.bias_wave = band == 0 && s.nb4 > 0 && tid < 64;
  o.bias_lane = o.bias_wave && tid < kTileCols / 4;
  o.qb = o.c0 / 4 + min(tid, kTileCols / 4 - 1);
  return o;
}

// Ordered sums dst = scale * sum_{i<n} src[i*stride], one thread each.
struct OrderedSums {
  const float* src[kMaxOrderedSums];
  int n[kMaxOrderedSums], stride[kMaxOrderedSums];
  float scale[kMaxOrderedSums];
  float* dst[kMaxOrderedSums];
  int count;
};
// Every term of a sum of at most kSumLds terms is staged in LDS (one memory
// round trip for all of them, overlapping the caller's own loads), then,
// after a barrier of the caller's, one thread adds them in order.
__device__ __forceinline__ void stage_sums(const OrderedSums& s, float (*terms)[kSumLds]) {
#pragma unroll
  for (int k = 0; k < kMaxOrderedSums; ++k)
    if (k < s.count && s.n[k] <= kSumLds)
      for (int i = threadIdx.x; i < s.n[k]; i += kOptThreads) terms[k][i] = s.src[k][long(i) * s.stride[k]];
}
__device__ __forceinline__ void ordered_sums(const OrderedSums& s, const float (*terms)[kSumLds]) {
  const int k = int(threadIdx.x);
  if (k >= s.count || k >= kMaxOrderedSums) return;
  const float* src = s.src[k];
  const int n = s.n[k], st = s.stride[k];
  float t = 0.f;
  if (n <= kSumLds) {
    for (int i = 0; i < n; ++i) t += terms[k][i];  // in order: the same sum on every run
  } else {
#pragma unroll 8
    for (int i = 0; i < n; ++i) t += src[long(i) * st];
  }
  *s.dst[k] = t * s.scale[k];
}

// The finish of a step: the sum of the workgroups' partials of g^2 (each
// thread a strided share, then the fixed-order block sum), the update count
// advanced, the ordered sums formed.  `terms` stages the sums' terms.
__device__ __forceinline__ void finish_step(const float* __restrict__ partials, int nparts, int* __restrict__ step,
                                            float* __restrict__ out, int accumulate, const OrderedSums& sums,
                                            float (*terms)[kSumLds], float* red) {
  stage_sums(sums, terms);
  float s = 0.f;
  for (int i = threadIdx.x; i < nparts; i += kOptThreads) s += partials[i];
  const float tot = block_sum<kOptThreads>(s, red);
  if (threadIdx.x == 0) {
    if (out) *out = accumulate ? *out + tot : tot;
    if (step) *step = *step + 1;
  }
  ordered_sums(sums, terms);
}

struct AdamSrcArgs {
  float* p;
  float* g;
  float* S;
  float* V;
  long n;
  int* step;
  float lr, b1, b2, eps, wd;
  float* partials;
  int nsrc;
  GradSrc src[kMaxGradSources];
  int plain0, plain_blocks;
  long plain4;  // float4s no source owns
  int nholes;   // the sources' float4 ranges [lo, hi), ascending and disjoint
  long hole_lo[2 * kMaxGradSources], hole_hi[2 * kMaxGradSources];
};

// Blocks [0, plain0) form the sources' gradients (source k owns blocks
// [block0, block0 + blocks)) and update their parameters; the rest run the
// grid-stride update over the float4s no source owns, numbered densely: j
// maps to arena float4 j plus the lengths of the holes at or below it.
// Block b's partial sum of g^2 goes to partials[b].
// STORE: the sources' formed gradients are written into g as well.
template <bool STORE>
__global__ __launch_bounds__(kOptThreads) __attribute__((amdgpu_waves_per_eu(4))) void k_adam_src(AdamSrcArgs a) {
  __shared__ float red[kOptThreads / 64];
  __shared__ float us[kOuterULds], vs[kOuterLds];
  // the update count before any other load, through the scalar cache (one
  // read per wavefront of one word every workgroup reads; no store of this
  // launch reaches it): thread 0, forming the step's scalars from it, then
  // waits for none of the vector loads
  typedef __attribute__((address_space(1))) const int global_int;
  const int stepc = *(global_int*)a.step;
  warm_kernargs<int(sizeof(AdamSrcArgs))>();
  const int blk = int(blockIdx.x);
  float alpha_t, eps_t;
  float gsq = 0.f;
  f32x4* P = reinterpret_cast<f32x4*>(a.p);
  f32x4* Gd = reinterpret_cast<f32x4*>(a.g);
  f32x4* Sv = reinterpret_cast<f32x4*>(a.S);
  f32x4* Vv = reinterpret_cast<f32x4*>(a.V);
  if (blk < a.plain0) {
    int k = 0;
#pragma unroll
    for (int i = 1; i < kMaxGradSources; ++i)
      if (i < a.nsrc && blk >= a.src[i].block0) k = i;
    const GradSrc& s = a.src[k];
    if (s.tiled) {
      // a tile (kTileOuts float4s per thread, both slices staged), in the
      // first row band with the bias's float4s of its columns
      const TileSpot t = tile_spot(s, xcd_tile(blk, s.block0, s.blocks));
      // the operand slices' loads first, then the parameters' and moments',
      // all in flight while the scalars are formed (unconditional, so that
      // thread 0's wait for the count waits for none of them; a row past the
      // block reads the block's first float4 and stores nothing)
      const OuterTileLoads tl = issue_outer_tile(s, t.r0, t.c0);
      long i[kTileOuts];
      f32x4 pv[kTileOuts], sv[kTileOuts], vv[kTileOuts];
#pragma unroll
      for (int o = 0; o < kTileOuts; ++o) {
        i[o] = s.w4 + t.q[o];
        const long il = t.ok[o] ? i[o] : s.w4;
        pv[o] = P[il];
        sv[o] = Sv[il];
        vv[o] = Vv[il];
      }
      // (left unset on waves that do not step the bias: a zero there would
      // cost a copy that waits for the loads)
      const long ib = s.b4 + t.qb;
      f32x4 pb, sb, vb;
      if (t.bias_wave) {
        pb = P[ib];
        sb = Sv[ib];
        vb = Vv[ib];
      }
      adam_scalars_of(stepc, a.lr, a.b1, a.b2, a.eps, &alpha_t, &eps_t);
      commit_outer_tile(tl, us, vs);
      f32x4 gv[kTileOuts];
      outer_grad_tile(us, vs, t.tr, t.tc4, gv);
#pragma unroll
      for (int o = 0; o < kTileOuts; ++o) {
        if (t.ok[o]) {
          if (STORE) Gd[i[o]] = gv[o];
          adam4(pv[o], gv[o], sv[o], vv[o], a.b1, a.b2, a.wd, eps_t, alpha_t, gsq);
          P[i[o]] = pv[o];
          Sv[i[o]] = sv[o];
          Vv[i[o]] = vv[o];
        }
      }
      if (t.bias_lane) {
        const f32x4 gb = outer_bias_tile(vs, t.tc4);
        if (STORE) Gd[ib] = gb;
        adam4(pb, gb, sb, vb, a.b1, a.b2, a.wd, eps_t, alpha_t, gsq);
        P[ib] = pb;
        Sv[ib] = sb;
        Vv[ib] = vb;
      }
      const float tot = block_sum<kOptThreads>(gsq, red);
      if (threadIdx.x == 0) a.partials[blk] = tot;
      return;
    }
    const int qb0 = (blk - s.block0) * kOptThreads;
    const OuterSlice o = outer_slice(s, qb0);  // uniform over the workgroup
    const bool staged = o.staged && s.blocks * kOptThreads >= s.nw4 + s.nb4;  // one float4 per thread
    const int nq = s.nw4 + s.nb4;
    const int step = s.blocks * kOptThreads;
    int q = qb0 + int(threadIdx.x);
    // the first float4's parameters and moments in flight while the
    // gradient's operands are staged and the scalars formed (unconditional,
    // as in the tiles; a thread past the source reads its last float4)
    auto where = [&](int qv) { return qv >= s.nw4 ? s.b4 + (qv - s.nw4) : s.w4 + qv; };
    f32x4 pv, sv, vv;
    {
      const long i = where(min(q, nq - 1));
      pv = P[i];
      sv = Sv[i];
      vv = Vv[i];
    }
    // a staged slice of one chunk in flight too while thread 0 forms the
    // scalars (the branches are uniform over the workgroup; a split-K
    // source's partials are loaded after them: held across the scalars'
    // arithmetic they would not fit the registers)
    if (staged && s.batch <= kOuterChunk) {
      const StageLoads sl = issue_stage(s, o);
      adam_scalars_of(stepc, a.lr, a.b1, a.b2, a.eps, &alpha_t, &eps_t);
      commit_stage(s, o, sl, us, vs);
    } else {
      if (staged) stage_outer(s, o, us, vs);
      adam_scalars_of(stepc, a.lr, a.b1, a.b2, a.eps, &alpha_t, &eps_t);
    }
    for (bool first = true; q < nq; q += step, first = false) {
      bool bias;
      int qq;
      const f32x4 gv = staged ? outer_grad_staged(s, o, us, vs, q, &bias, &qq) : source_grad(s, q, &bias, &qq);
      const long i = (bias ? s.b4 : s.w4) + qq;
      if (!first) {
        pv = P[i];
        sv = Sv[i];
        vv = Vv[i];
      }
      if (STORE) Gd[i] = gv;
      adam4(pv, gv, sv, vv, a.b1, a.b2, a.wd, eps_t, alpha_t, gsq);
      P[i] = pv;
      Sv[i] = sv;
      Vv[i] = vv;
    }
  } else {
    const long n4 = a.n / 4;
    const long stride = long(a.plain_blocks) * kOptThreads;
    adam_loop(a.p, a.g, a.S, a.V, long(blk - a.plain0) * kOptThreads + threadIdx.x, a.plain4, stride, a.step, a.lr,
              a.b1, a.b2, a.eps, a.wd, gsq, &alpha_t, &eps_t, [&](long j) {
                long i = j;
#pragma unroll
                for (int h = 0; h < 2 * kMaxGradSources; ++h)
                  if (h < a.nholes && i >= a.hole_lo[h]) i += a.hole_hi[h] - a.hole_lo[h];
                return i;
              });
    // Tail (n % 4) handled by the first plain block; no source reaches it.
    if (blk == a.plain0) {
      for (long i = n4 * 4 + threadIdx.x; i < a.n; i += kOptThreads) {
#pragma clang fp contract(off)
        const float graw = a.g[i];
        gsq += graw * graw;
        const float gg = a.wd != 0.f ? graw + a.wd * a.p[i] : graw;
        a.V[i] = gg * gg + a.b2 * a.V[i];
        a.S[i] = gg + a.b1 * a.S[i];
        a.p[i] = a.p[i] - (a.S[i] / (sqrtf(a.V[i]) + eps_t)) * alpha_t;
      }
    }
  }
  const float tot = block_sum<kOptThreads>(gsq, red);
  if (threadIdx.x == 0) a.partials[blk] = tot;
}

// Writes the sources' gradients only (no step).
struct SrcSet {
  int nsrc;
  GradSrc src[kMaxGradSources];
};
__global__ __launch_bounds__(kOptThreads) void k_sources_write(SrcSet a) {
  warm_kernargs<int(sizeof(SrcSet))>();
  const int blk = int(blockIdx.x);
  int k = 0;
#pragma unroll
  for (int i = 1; i < kMaxGradSources; ++i)
    if (i < a.nsrc && blk >= a.src[i].block0) k = i;
  const GradSrc& s = a.src[k];
  __shared__ float us[kOuterULds], vs[kOuterLds];
  if (s.tiled) {
    const TileSpot t = tile_spot(s, xcd_tile(blk, s.block0, s.blocks));
    commit_outer_tile(issue_outer_tile(s, t.r0, t.c0), us, vs);
    f32x4 gv[kTileOuts];
    outer_grad_tile(us, vs, t.tr, t.tc4, gv);
#pragma unroll
    for (int o = 0; o < kTileOuts; ++o)
      if (t.ok[o]) reinterpret_cast<f32x4*>(s.gw)[t.q[o]] = gv[o];
    if (t.bias_lane) reinterpret_cast<f32x4*>(s.gb)[t.qb] = outer_bias_tile(vs, t.tc4);
    return;
  }
  const int qb0 = (blk - s.block0) * kOptThreads;
  const OuterSlice o = outer_slice(s, qb0);
  const int nq = s.nw4 + s.nb4;
  const bool staged = o.staged && s.blocks * kOptThreads >= nq;
  if (staged) stage_outer(s, o, us, vs);
  for (int q = qb0 + int(threadIdx.x); q < nq; q += s.blocks * kOptThreads) {
    bool bias;
    int qq;
    const f32x4 gv = staged ? outer_grad_staged(s, o, us, vs, q, &bias, &qq) : source_grad(s, q, &bias, &qq);
    if (!bias) {
      reinterpret_cast<f32x4*>(s.gw)[qq] = gv;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (4 * qq + j < s.cols) s.gb[4 * qq + j] = gv[j];
    }
  }
}

// The finish of a step as a launch of its own (ttrl_ordered_sums), the
// sums' terms staged while the partials are read.
__global__ __launch_bounds__(kOptThreads) void k_finish_sums(const float* __restrict__ partials, int nparts,
                                                             int* __restrict__ step, float* __restrict__ out,
                                                             int accumulate, OrderedSums sums) {
  __shared__ float red[kOptThreads / 64];
  __shared__ float terms[kMaxOrderedSums][kSumLds];
  warm_kernargs<int(sizeof(OrderedSums) + 40)>();
  finish_step(partials, nparts, step, out, accumulate, sums, terms, red);
}

__global__ __launch_bounds__(kOptThreads) void k_sumsq(const float* __restrict__ x, long n,
                                                       float* __restrict__ partials) {
  __shared__ float red[kOptThreads / 64];
  float s = 0.f;
  const long stride = long(gridDim.x) * kOptThreads;
  for (long i = blockIdx.x * long(kOptThreads) + threadIdx.x; i < n; i += stride) {
    const float v = x[i];
    s += v * v;
  }
  const float tot = block_sum<kOptThreads>(s, red);
  if (threadIdx.x == 0) partials[blockIdx.x] = tot;
}

__global__ __launch_bounds__(kOptThreads) void k_polyak(float* __restrict__ dst, const float* __restrict__ src,
                                                        long n, float keep, float tau) {
  const long stride = long(gridDim.x) * kOptThreads;
  for (long i = blockIdx.x * long(kOptThreads) + threadIdx.x; i < n; i += stride) {
    dst[i] = dst[i] * keep + src[i] * tau;
  }
}

__global__ __launch_bounds__(kOptThreads) void k_fill(float* __restrict__ p, long n, float v) {
  const long stride = long(gridDim.x) * kOptThreads;
  for (long i = blockIdx.x * long(kOptThreads) + threadIdx.x; i < n; i += stride) p[i] = v;
}

__global__ void k_fill_i32(int* __restrict__ p, long n, int v) {
  for (long i = blockIdx.x * long(blockDim.x) + threadIdx.x; i < n; i += long(gridDim.x) * blockDim.x) p[i] = v;
}

inline unsigned grid_for(long n, long per_thread = 1) {
  long b = (n / per_thread + kOptThreads - 1) / kOptThreads;
  if (b < 1) b = 1;
  if (b > kOptMaxBlocks) b = kOptMaxBlocks;
  return unsigned(b);
}

// Scratch of the allocation-free Adam step: one partial sum of squared
// gradients per workgroup of k_adam.  A launch uses at most kOptMaxBlocks
// workgroups, so this bounds nothing about n.  Each GPU holds its own copy;
// host code reaches it only through the address hipGetSymbolAddress gives
// for the current device (static_scratch_for), never through the name.
constexpr int kStaticScratchFloats = kOptMaxBlocks;
__device__ __align__(256) float scratch[kStaticScratchFloats];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on the current device, resolved once per
// device (with that device current) and kept.
int static_scratch_for(float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_error(e, "hipGetDevice (ttrl_adam_step_static)");
  if (dev < 0 || dev >= kMaxDevices)
    return set_error(TTRL_EINVAL, "ttrl_adam_step_static: device %d beyond the %d supported", dev, kMaxDevices);
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) return hip_error(e, "hipGetSymbolAddress (ttrl_adam_step_static scratch)");
    g_scratch_ptr[dev] = static_cast<float*>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return TTRL_OK;
}

int check_adam_args(const float* p, const float* g, const float* m_s, const float* v_s, long n, const int* step,
                    float lr, float beta1, float beta2, float eps, float weight_decay, const char* name) {
  TTRL_REQUIRE(p && g && m_s && v_s && step, "%s: null argument", name);
  TTRL_REQUIRE(n > 0, "%s: empty parameter range", name);
  TTRL_REQUIRE(lr > 0.f && eps > 0.f && beta1 >= 0.f && beta1 < 1.f && beta2 >= 0.f && beta2 < 1.f &&
                   weight_decay >= 0.f,
               "%s: bad hyper-parameters", name);
  TTRL_REQUIRE(((reinterpret_cast<uintptr_t>(p) | reinterpret_cast<uintptr_t>(g) |
                 reinterpret_cast<uintptr_t>(m_s) | reinterpret_cast<uintptr_t>(v_s)) & 15) == 0,
               "%s: buffers must be 16-byte aligned", name);
  return TTRL_OK;
}

inline bool inside(const float* x, long count, const float* base, long n) {
  return x >= base && x + count <= base + n;
}
inline bool aligned16(const void* x) { return (reinterpret_cast<uintptr_t>(x) & 15) == 0; }

// Checks sources[0 .. n) and fills their device form; blocks are laid out
// from block 0.  With an arena (g, gn), each written range must lie inside
// it, and ranges of different sources must not overlap.  Sources of kind
// TTRL_GRAD_NONE are skipped.  *blocks receives the blocks they use.
int make_sources(int n, const ttrl_grad_source* srcs, const float* g, long gn, GradSrc* out, int* count, int* blocks,
                 const char* name) {
  TTRL_REQUIRE(n >= 0 && n <= kMaxGradSources && (n == 0 || srcs), "%s: %d sources outside [0, %d]", name, n,
               kMaxGradSources);
  int c = 0, b = 0;
  std::vector<std::pair<const float*, const float*>> spans;
  for (int i = 0; i < n; ++i) {
    const ttrl_grad_source& s = srcs[i];
    if (s.kind == TTRL_GRAD_NONE) continue;
    TTRL_REQUIRE(s.kind == TTRL_GRAD_SPLITS || s.kind == TTRL_GRAD_OUTER, "%s: source %d: unknown kind %d", name, i,
                 s.kind);
    TTRL_REQUIRE(s.rows > 0 && s.cols > 0 && (long(s.rows) * s.cols) % 4 == 0 && long(s.rows) * s.cols < (1L << 30),
                 "%s: source %d: a %dx%d block (rows * cols must be a positive multiple of 4)", name, i, s.rows,
                 s.cols);
    TTRL_REQUIRE(s.dw && aligned16(s.dw) && (!s.db || aligned16(s.db)),
                 "%s: source %d: gradient destinations must be 16-byte aligned", name, i);
    const long wn = long(s.rows) * s.cols, bn = s.db ? (s.cols + 3) / 4 * 4 : 0;
    if (g) {
      TTRL_REQUIRE(inside(s.dw, wn, g, gn) && (!s.db || inside(s.db, bn, g, gn)),
                   "%s: source %d: gradient outside the arena", name, i);
    }
    spans.emplace_back(s.dw, s.dw + wn);
    if (s.db) spans.emplace_back(s.db, s.db + bn);
    GradSrc d{};
    d.kind = s.kind;
    d.rows = s.rows;
    d.cols = s.cols;
    d.gw = s.dw;
    d.gb = s.db;
    d.w4 = g ? (s.dw - g) / 4 : 0;
    d.b4 = g && s.db ? (s.db - g) / 4 : -1;
    d.nw4 = int(wn / 4);
    d.nb4 = int(bn / 4);
    d.dc.set(s.cols);
    if (s.kind == TTRL_GRAD_SPLITS) {
      TTRL_REQUIRE(s.part && aligned16(s.part) && s.splits >= 1 && s.cols % 4 == 0,
                   "%s: source %d: split partials need a 16-byte aligned buffer, splits >= 1 and cols %% 4 == 0",
                   name, i);
      d.part = s.part;
      d.splits = s.splits;
      d.sstride = (long(s.rows) + (s.db ? 1 : 0)) * s.cols;
      d.scale = s.scale;
      d.bias_scale = s.bias_scale;
    } else {
      TTRL_REQUIRE(s.u && s.v && s.batch >= 1, "%s: source %d: an outer product needs u, v and batch >= 1", name, i);
      d.u = s.u;
      d.v = s.v;
      d.batch = s.batch;
      // wide enough that one row band of v would not fit in LDS: by tiles
      d.tiled = s.cols % kTileCols == 0 && s.batch <= kTileBatch && aligned16(s.v) && s.batch * s.cols > kOuterLds;
      if (d.tiled) {
        d.ntc = s.cols / kTileCols;
        d.ntiles = int(ceil_div(long(s.rows), kTileRows)) * d.ntc;
      }
    }
    d.blocks = d.tiled ? d.ntiles : int(ceil_div(long(d.nw4) + d.nb4, kOptThreads));
    out[c++] = d;
  }
  // Workgroups are dispatched in block order and a launch's whole grid is
  // resident at once, so a workgroup's loads queue behind those of the
  // blocks before it.  The few workgroups of the staged outer products (a
  // staging round trip, then the product) and of the split-K sources (a
  // batch of partials per float4) are the longest chains: they take the
  // first blocks, the many short tile chains the last.
  auto chain = [](const GradSrc& s) { return s.kind == TTRL_GRAD_SPLITS ? 1 : s.tiled ? 2 : 0; };
  std::stable_sort(out, out + c, [&](const GradSrc& x, const GradSrc& y) { return chain(x) < chain(y); });
  for (int k = 0; k < c; ++k) {
    out[k].block0 = b;
    b += out[k].blocks;
  }
  std::sort(spans.begin(), spans.end());
  for (size_t i = 1; i < spans.size(); ++i)
    TTRL_REQUIRE(spans[i].first >= spans[i - 1].second, "%s: two sources write the same gradient", name);
  *count = c;
  *blocks = b;
  return TTRL_OK;
}

int make_sums(int n, const ttrl_ordered_sum* sums, OrderedSums* out, const char* name) {
  TTRL_REQUIRE(n >= 0 && n <= kMaxOrderedSums && (n == 0 || sums), "%s: %d ordered sums outside [0, %d]", name, n,
               kMaxOrderedSums);
  *out = OrderedSums{};
  for (int i = 0; i < n; ++i) {
    TTRL_REQUIRE(sums[i].src && sums[i].dst && sums[i].n >= 1 && sums[i].stride >= 1,
                 "%s: ordered sum %d: null buffer, empty or bad stride", name, i);
    for (int j = 0; j < i; ++j)
      TTRL_REQUIRE(sums[j].dst != sums[i].dst, "%s: ordered sums %d and %d write the same value", name, j, i);
    out->src[i] = sums[i].src;
    out->n[i] = sums[i].n;
    out->stride[i] = sums[i].stride;
    out->scale[i] = sums[i].scale;
    out->dst[i] = sums[i].dst;
  }
  out->count = n;
  return TTRL_OK;
}

}  // namespace ttrl

using namespace ttrl;

extern "C" {

int ttrl_adam_step_sources(ttrl_ctx* ctx, const ttrl_adam_sources_desc* d) {
  TTRL_REQUIRE(ctx && d, "ttrl_adam_step_sources: null argument");
  int rc = check_adam_args(d->p, d->g, d->m_s, d->v_s, d->n, d->step, d->lr, d->beta1, d->beta2, d->eps,
                           d->weight_decay, "ttrl_adam_step_sources");
  if (rc) return rc;
  AdamSrcArgs a{};
  int srcblocks = 0;
  rc = make_sources(d->nsources, d->sources, d->g, d->n, a.src, &a.nsrc, &srcblocks, "ttrl_adam_step_sources");
  if (rc) return rc;
  OrderedSums sums;
  rc = make_sums(d->nsums, d->sums, &sums, "ttrl_adam_step_sources");
  if (rc) return rc;
  a.p = d->p;
  a.g = d->g;
  a.S = d->m_s;
  a.V = d->v_s;
  a.n = d->n;
  a.step = d->step;
  a.lr = d->lr;
  a.b1 = d->beta1;
  a.b2 = d->beta2;
  a.eps = d->eps;
  a.wd = d->weight_decay;
  a.plain0 = srcblocks;
  std::vector<std::pair<long, long>> holes;
  for (int k = 0; k < a.nsrc; ++k) {
    holes.emplace_back(a.src[k].w4, a.src[k].w4 + a.src[k].nw4);
    if (a.src[k].nb4 > 0) holes.emplace_back(a.src[k].b4, a.src[k].b4 + a.src[k].nb4);
  }
  std::sort(holes.begin(), holes.end());  // disjoint (make_sources checked)
  a.nholes = int(holes.size());
  a.plain4 = d->n / 4;
  for (int h = 0; h < a.nholes; ++h) {
    a.hole_lo[h] = holes[h].first;
    a.hole_hi[h] = holes[h].second;
    a.plain4 -= holes[h].second - holes[h].first;
  }
  // the plain part: a float4 per thread, within what the source workgroups
  // leave of a launch's kOptMaxBlocks (so the whole grid is resident at
  // once), and one workgroup at least (the tail of n % 4 and its g^2)
  a.plain_blocks = std::max(1, std::min(int(grid_for(a.plain4 * 4, 4)), kOptMaxBlocks - srcblocks));
  const int blocks = a.plain0 + a.plain_blocks;
  long wsf = 0;
  a.partials = ctx_workspace(ctx, &wsf);
  TTRL_REQUIRE(wsf >= long(blocks), "ttrl_adam_step_sources: workspace too small");
  hipStream_t st = stream_of(ctx);
  if (d->store_grads)
    hipLaunchKernelGGL(k_adam_src<true>, dim3(unsigned(blocks)), dim3(kOptThreads), 0, st, a);
  else
    hipLaunchKernelGGL(k_adam_src<false>, dim3(unsigned(blocks)), dim3(kOptThreads), 0, st, a);
  hipLaunchKernelGGL(k_finish_sums, dim3(1), dim3(kOptThreads), 0, st, a.partials, blocks, d->step, d->grad_sq,
                     d->accumulate_grad_sq, sums);
  return check_launch("ttrl_adam_step_sources");
}

int ttrl_grad_sources_materialize(ttrl_ctx* ctx, int n, const ttrl_grad_source* sources) {
  TTRL_REQUIRE(ctx, "ttrl_grad_sources_materialize: null ctx");
  SrcSet a{};
  int blocks = 0;
  int rc = make_sources(n, sources, nullptr, 0, a.src, &a.nsrc, &blocks, "ttrl_grad_sources_materialize");
  if (rc) return rc;
  if (blocks == 0) return TTRL_OK;
  hipLaunchKernelGGL(k_sources_write, dim3(unsigned(blocks)), dim3(kOptThreads), 0, stream_of(ctx), a);
  return check_launch("ttrl_grad_sources_materialize");
}

int ttrl_ordered_sums(ttrl_ctx* ctx, int n, const ttrl_ordered_sum* sums) {
  TTRL_REQUIRE(ctx, "ttrl_ordered_sums: null ctx");
  OrderedSums s;
  int rc = make_sums(n, sums, &s, "ttrl_ordered_sums");
  if (rc) return rc;
  if (n == 0) return TTRL_OK;
  hipLaunchKernelGGL(k_finish_sums, dim3(1), dim3(kOptThreads), 0, stream_of(ctx), (const float*)nullptr, 0,
                     (int*)nullptr, (float*)nullptr, 0, s);
  return check_launch("ttrl_ordered_sums");
}

int ttrl_adam_step(ttrl_ctx* ctx, float* p, const float* g, float* m_s, float* v_s, long n, int* step, float lr,
                   float beta1, float beta2, float eps, float weight_decay, float* grad_sq, int accumulate_grad_sq) {
  TTRL_REQUIRE(ctx, "ttrl_adam_step: null ctx");
  int rc = check_adam_args(p, g, m_s, v_s, n, step, lr, beta1, beta2, eps, weight_decay, "ttrl_adam_step");
  if (rc) return rc;
  long wsf = 0;
  float* ws = ctx_workspace(ctx, &wsf);
  const unsigned blocks = grid_for(n, 4);
  TTRL_REQUIRE(wsf >= long(blocks), "ttrl_adam_step: workspace too small");
  hipStream_t st = stream_of(ctx);
  hipLaunchKernelGGL(k_adam, dim3(blocks), dim3(kOptThreads), 0, st, p, g, m_s, v_s, n, step, lr, beta1, beta2,
                     eps, weight_decay, ws);
  hipLaunchKernelGGL(k_finish, dim3(1), dim3(kOptThreads), 0, st, ws, int(blocks), step, grad_sq,
                     accumulate_grad_sq);
  return check_launch("ttrl_adam_step");
}

}  // extern "C"

namespace {
// The clipped step's launches; the finishing one also ends a learner step
// when `end` names its metric ring (counter non-null).
struct StepEnd {
  int* counter;
  const float* metrics;
  int n;
  float* ring;
  int slots;
};
int adam_step_clipped(ttrl_ctx* ctx, float* p, float* g, float* m_s, float* v_s, long n, int* step, float lr,
                      float beta1, float beta2, float eps, float weight_decay, float* grad_sq, int accumulate_grad_sq,
                      float max_norm, float* sq_out, float* norm_out, const StepEnd& end, const char* name) {
  TTRL_REQUIRE(ctx, "%s: null ctx", name);
  int rc = check_adam_args(p, g, m_s, v_s, n, step, lr, beta1, beta2, eps, weight_decay, name);
  if (rc) return rc;
  TTRL_REQUIRE(max_norm > 0.f, "%s: max_norm must be > 0, got %g", name, double(max_norm));
  // the norm's partial sums as ttrl_sum_squares forms them, so every
  // workgroup's sum is the one ttrl_clip_grad_norm forms
  long wsf = 0;
  float* ws = ctx_workspace(ctx, &wsf);
  const unsigned blocks = grid_for(n, 4), sq_blocks = grid_for(n, 4);
  TTRL_REQUIRE(wsf >= long(blocks) + sq_blocks, "%s: workspace too small", name);
  float* sq_parts = ws + blocks;
  hipStream_t st = stream_of(ctx);
  hipLaunchKernelGGL(k_sumsq, dim3(sq_blocks), dim3(kOptThreads), 0, st, g, n, sq_parts);
  hipLaunchKernelGGL(k_adam_clip, dim3(blocks), dim3(kOptThreads), 0, st, p, g, m_s, v_s, n, step, lr, beta1, beta2,
                     eps, weight_decay, ws, ClipScale{sq_parts, int(sq_blocks), max_norm, sq_out, norm_out});
  if (end.counter)
    hipLaunchKernelGGL(k_finish_end, dim3(1), dim3(kOptThreads), 0, st, ws, int(blocks), step, grad_sq,
                       accumulate_grad_sq, end.counter, end.metrics, end.n, end.ring, end.slots);
  else
    hipLaunchKernelGGL(k_finish, dim3(1), dim3(kOptThreads), 0, st, ws, int(blocks), step, grad_sq,
                       accumulate_grad_sq);
  return check_launch(name);
}
}  // namespace

extern "C" {

int ttrl_adam_step_clipped(ttrl_ctx* ctx, float* p, float* g, float* m_s, float* v_s, long n, int* step,
                           float lr, float beta1, float beta2, float eps, float weight_decay, float* grad_sq,
                           int accumulate_grad_sq, float max_norm, float* sq_out, float* norm_out) {
  return adam_step_clipped(ctx, p, g, m_s, v_s, n, step, lr, beta1, beta2, eps, weight_decay, grad_sq,
                           accumulate_grad_sq, max_norm, sq_out, norm_out, StepEnd{}, "ttrl_adam_step_clipped");
}

int ttrl_adam_step_clipped_end(ttrl_ctx* ctx, float* p, float* g, float* m_s, float* v_s, long n, int* step,
                               float lr, float beta1, float beta2, float eps, float weight_decay, float* grad_sq,
                               int accumulate_grad_sq, float max_norm, float* sq_out, float* norm_out, int* counter,
                               const float* metrics, int n_metrics, float* ring, int slots) {
  TTRL_REQUIRE(counter, "ttrl_adam_step_clipped_end: null counter");
  TTRL_REQUIRE(n_metrics >= 0 && slots >= 0 && (n_metrics == 0 || (metrics && ring)),
               "ttrl_adam_step_clipped_end: bad metric ring");
  return adam_step_clipped(ctx, p, g, m_s, v_s, n, step, lr, beta1, beta2, eps, weight_decay, grad_sq,
                           accumulate_grad_sq, max_norm, sq_out, norm_out,
                           StepEnd{counter, metrics, n_metrics, ring, slots}, "ttrl_adam_step_clipped_end");
}

int ttrl_adam_step_static(void* stream, float* p, const float* g, float* m_s, float* v_s, long n, int* step,
                          float lr, float beta1, float beta2, float eps, float weight_decay, float* grad_sq,
                          int accumulate_grad_sq) {
  int rc = check_adam_args(p, g, m_s, v_s, n, step, lr, beta1, beta2, eps, weight_decay, "ttrl_adam_step_static");
  if (rc) return rc;
  const unsigned blocks = grid_for(n, 4);
  TTRL_REQUIRE(blocks <= unsigned(kStaticScratchFloats),
               "ttrl_adam_step_static: %u workgroups exceed the %d partial sums of the static scratch", blocks,
               kStaticScratchFloats);
  float* partials = nullptr;
  rc = static_scratch_for(&partials);
  if (rc) return rc;
  // Every workgroup writes its own partial before k_finish reads them, so
  // nothing in the scratch needs clearing between calls.
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(k_adam, dim3(blocks), dim3(kOptThreads), 0, st, p, g, m_s, v_s, n, step, lr, beta1, beta2,
                     eps, weight_decay, partials);
  hipLaunchKernelGGL(k_finish, dim3(1), dim3(kOptThreads), 0, st, partials, int(blocks), step, grad_sq,
                     accumulate_grad_sq);
  return check_launch("ttrl_adam_step_static");
}

int ttrl_adam_step_deferred(ttrl_ctx* ctx, float* p, const float* g, float* m_s, float* v_s, long n,
                            const int* step, float lr, float beta1, float beta2, float eps, float weight_decay,
                            int slot) {
  TTRL_REQUIRE(ctx, "ttrl_adam_step_deferred: null ctx");
  int rc = check_adam_args(p, g, m_s, v_s, n, step, lr, beta1, beta2, eps, weight_decay, "ttrl_adam_step_deferred");
  if (rc) return rc;
  TTRL_REQUIRE(slot >= 0 && slot < kAdamSlots, "ttrl_adam_step_deferred: slot %d outside [0, %d)", slot,
               kAdamSlots);
  static_assert(kAdamSlotFloats >= kOptMaxBlocks, "a slot holds one launch's partials");
  hipLaunchKernelGGL(k_adam, dim3(grid_for(n, 4)), dim3(kOptThreads), 0, stream_of(ctx), p, g, m_s, v_s, n, step,
                     lr, beta1, beta2, eps, weight_decay, ctx_adam_partials(ctx) + long(slot) * kAdamSlotFloats);
  return check_launch("ttrl_adam_step_deferred");
}

int ttrl_adam_multi(ttrl_ctx* ctx, int nranges, const ttrl_adam_range* ranges, float* polyak_dst,
                    const float* polyak_src, long polyak_n, float tau) {
  TTRL_REQUIRE(ctx, "ttrl_adam_multi: null ctx");
  TTRL_REQUIRE(nranges >= 0 && nranges <= kMultiRanges && (nranges == 0 || ranges),
               "ttrl_adam_multi: %d ranges outside [0, %d]", nranges, kMultiRanges);
  TTRL_REQUIRE(polyak_n >= 0 && (polyak_n == 0 || (polyak_dst && polyak_src)),
               "ttrl_adam_multi: null Polyak buffer");
  TTRL_REQUIRE(tau >= 0.f && tau <= 1.f, "ttrl_adam_multi: tau must be in [0, 1]");
  AdamMulti a{};
  a.nr = nranges;
  int blocks = 0;
  bool slot_used[kAdamSlots] = {};
  for (int i = 0; i < nranges; ++i) {
    const ttrl_adam_range& r = ranges[i];
    int rc = check_adam_args(r.p, r.g, r.m_s, r.v_s, r.n, r.step, r.lr, r.beta1, r.beta2, r.eps, r.weight_decay,
                             "ttrl_adam_multi");
    if (rc) return rc;
    TTRL_REQUIRE(r.slot >= 0 && r.slot < kAdamSlots && !slot_used[r.slot],
                 "ttrl_adam_multi: range %d: slot %d outside [0, %d) or taken twice", i, r.slot, kAdamSlots);
    slot_used[r.slot] = true;
    const int nb = int(grid_for(r.n, 4));
    a.r[i] = AdamRange{r.p, r.g, r.m_s, r.v_s, r.n, r.step, r.lr, r.beta1, r.beta2, r.eps, r.weight_decay,
                       ctx_adam_partials(ctx) + long(r.slot) * kAdamSlotFloats, blocks, nb};
    blocks += nb;
  }
  a.pd = polyak_dst;
  a.ps = polyak_src;
  a.pn = polyak_n;
  a.keep = 1.f - tau;
  a.tau = tau;
  a.pblock0 = blocks;
  a.pblocks = polyak_n > 0 ? int(grid_for(polyak_n)) : 0;
  blocks += a.pblocks;
  if (blocks == 0) return TTRL_OK;
  hipLaunchKernelGGL(k_adam_multi, dim3(unsigned(blocks)), dim3(kOptThreads), 0, stream_of(ctx), a);
  return check_launch("ttrl_adam_multi");
}

int ttrl_adam_finish_slots(ttrl_ctx* ctx, int n, const ttrl_adam_finish* f) {
  TTRL_REQUIRE(ctx && (n == 0 || f), "ttrl_adam_finish_slots: null argument");
  TTRL_REQUIRE(n >= 0 && n <= kAdamSlots, "ttrl_adam_finish_slots: %d finishes outside [0, %d]", n, kAdamSlots);
  if (n == 0) return TTRL_OK;
  FinishSlots fs{};
  for (int i = 0; i < n; ++i) {
    TTRL_REQUIRE(f[i].slot >= 0 && f[i].slot < kAdamSlots, "ttrl_adam_finish_slots: slot %d outside [0, %d)",
                 f[i].slot, kAdamSlots);
    TTRL_REQUIRE(f[i].n > 0 && f[i].step, "ttrl_adam_finish_slots: finish %d: empty range or null step", i);
    fs.parts[i] = ctx_adam_partials(ctx) + long(f[i].slot) * kAdamSlotFloats;
    TTRL_REQUIRE(f[i].parts >= 0 && f[i].parts <= kAdamSlotFloats,
                 "ttrl_adam_finish_slots: finish %d: %d partial sums outside [0, %d]", i, f[i].parts, kAdamSlotFloats);
    fs.count[i] = f[i].parts > 0 ? f[i].parts : int(grid_for(f[i].n, 4));
    fs.step[i] = f[i].step;
    fs.out[i] = f[i].grad_sq;
    fs.accumulate[i] = f[i].accumulate;
  }
  hipLaunchKernelGGL(k_finish_slots, dim3(unsigned(n)), dim3(kOptThreads), 0, stream_of(ctx), fs);
  return check_launch("ttrl_adam_finish_slots");
}

int ttrl_sum_squares(ttrl_ctx* ctx, const float* x, long n, float* out, int accumulate) {
  TTRL_REQUIRE(ctx && x && out, "ttrl_sum_squares: null argument");
  TTRL_REQUIRE(n >= 0, "ttrl_sum_squares: negative length");
  long wsf = 0;
  float* ws = ctx_workspace(ctx, &wsf);
  const unsigned blocks = grid_for(n > 0 ? n : 1, 4);
  hipStream_t st = stream_of(ctx);
  hipLaunchKernelGGL(k_sumsq, dim3(blocks), dim3(kOptThreads), 0, st, x, n, ws);
  hipLaunchKernelGGL(k_finish, dim3(1), dim3(kOptThreads), 0, st, ws, int(blocks), (int*)nullptr, out,
                     accumulate);
  return check_launch("ttrl_sum_squares");
}

int ttrl_polyak(ttrl_ctx* ctx, float* dst, const float* src, long n, float tau) {
  TTRL_REQUIRE(ctx && dst && src, "ttrl_polyak: null argument");
  TTRL_REQUIRE(tau >= 0.f && tau <= 1.f, "ttrl_polyak: tau must be in [0, 1]");
  if (n <= 0) return TTRL_OK;
  hipLaunchKernelGGL(k_polyak, dim3(grid_for(n)), dim3(kOptThreads), 0, stream_of(ctx), dst, src, n, 1.f - tau,
                     tau);
  return check_launch("ttrl_polyak");
}

int ttrl_fill_f32(ttrl_ctx* ctx, float* dst, float value, long n) {
  TTRL_REQUIRE(ctx && (dst || n == 0), "ttrl_fill_f32: null argument");
  if (n <= 0) return TTRL_OK;
  hipLaunchKernelGGL(k_fill, dim3(grid_for(n)), dim3(kOptThreads), 0, stream_of(ctx), dst, n, value);
  return check_launch("ttrl_fill_f32");
}

int ttrl_fill_i32(ttrl_ctx* ctx, int* dst, int value, long n) {
  TTRL_REQUIRE(ctx && (dst || n == 0), "ttrl_fill_i32: null argument");
  if (n <= 0) return TTRL_OK;
  hipLaunchKernelGGL(k_fill_i32, dim3(grid_for(n)), dim3(kOptThreads), 0, stream_of(ctx), dst, n, value);
  return check_launch("ttrl_fill_i32");
}

}  // extern "C"
