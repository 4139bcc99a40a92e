// The last two layers of the DQN update's Q networks, the loss and the
// head's backward in two launches (ttrl/algos/dqn/losses.py:77-140 over
// ttrl/nets/encoders.py's Linear(3136, 512) -> ReLU -> QHead Linear(512, A)).
//
// Launch 1, the first linear layer of every feature set, a GEMM on the
// MFMA core planned like any other; when its plan splits K the partial
// tiles stay in the workspace (run_gemm_deferred).
//
// Launch 2, k_dqn_tail, one workgroup per sample b:
//   h_g[b]  = relu(sum of the split partials in split order + b1_g)   (what
//             k_splitk_reduce would write; read back when K was not split)
//   q_g[b]  = h_g[b] W2_g + b2_g                 fixed-order block sums
//   the DQN row of sample b (dqn_row.hpp): a* from group 1, valued by group
//             G-1, Huber, IS weight, td_abs, dL/dq
//   dh[b]   = (dq[b] W2_0^T) * [h_0[b] > 0]      the gradient entering the
//             first layer's backward, already through its ReLU
// and the workgroup that finishes last (a device-scope counter, reset by it)
// sums, in sample order, the batch loss and mean Q and, when the caller asks
// for them here, the second layer's weight and bias gradients
// dW2 = h_0^T dq, db2 = column sums of dq.  A caller that leaves dW2 out
// forms it later from h_0 and dq (an outer-product gradient source of the
// optimizer step), off this kernel's serial last phase.
//
// This replaces a split-K reduce, the Q-head-and-loss kernel and the second
// layer's backward launch: three graph nodes become one.
#include "dqn_row.hpp"
#include "tile_gemm.hpp"

#include <algorithm>
#include <cmath>

namespace ttrl {
namespace {

constexpr int kTailThreads = 256;
constexpr int kTailMaxF = 2048;  // first-layer outputs per feature set held in LDS
constexpr int kTailMaxA = 32;
constexpr int kTailMaxB = kSyncPartials / 2;  // two partial sums per sample in the sync words
constexpr int kTailChunk = 32;                // samples per pass of the weight-gradient sum
constexpr int kTailItems = 8;                 // first-layer outputs per thread per pass
constexpr int kTailSplits = 16;               // split partials of an output loaded in one batch, at most
// The vector path (F % 4 == 0, aligned buffers, G F A <= kTailW2Lds): the
// split partials and biases read as float4s, kTailItems4 of them per thread
// per pass, and every set's second-layer weights staged in LDS by
// cooperative float4 loads, so that a thread's first round trip carries
// about 30 loads (a wavefront keeps at most 63 in flight; the scalar path's
// W2 rows and split partials are over 120 and take several trips).
constexpr int kTailItems4 = 2;
constexpr int kTailW2Lds = 3 * 512 * 8;
constexpr int kTailW2Loads = (kTailW2Lds / 4 + kTailThreads - 1) / kTailThreads;
static_assert(kSyncPartials + kTailChunk * kTailMaxA <= 3 * kTailMaxF, "the last workgroup's staging fits hs");

constexpr unsigned kFc1Cfgs = cfg_bit(T32x32) | cfg_bit(T64x32) | cfg_bit(T32x64) | cfg_bit(T64x64) |
                              cfg_bit(T32x32K2) | cfg_bit(T32x32K4) | cfg_bit(T64x32K2) | cfg_bit(T32x64K2);

struct TailArgs {
  int B, F, A, G, splits;  // splits 0: h holds the first layer's outputs already
  FDiv fdiv;               // division by F
  int fa4;                 // float4s of one set's W2 (vector path)
  FDiv fa4div;             // division by fa4
  const float* part;       // [G][splits][B][F]
  float* h[3];
  const float* b1[3];
  const float* W2[3];
  const float* b2[3];
  float* q[3];
  const float* onehot;
  const float* rewards;
  const float* dones;
  const float* discounts;
  const float* weights;
  float delta;
  float* loss;
  float* mean_q;
  float* td_abs;
  float* dq;
  float* next_act;
  float* td_target;
  float* dh;
  float* dW2;
  float* db2;
  float beta_w;
  unsigned* counter;
  float* partials;
  float* loss_terms;  // not null: per-sample terms for the caller, no batch phase
};

// Every phase issues all of its loads before it uses one: the kernel is a
// chain of memory round trips, one workgroup per sample, so the number of
// trips, not the arithmetic, sets its duration.  The inner loops carry no
// per-action or per-row branch (a guarded load or LDS read becomes a basic
// block of its own, with a wait of its own): action columns run to AP with
// clamped indexes or zero padding, and the extra accumulators are dropped.
// Sum of v over the 64 lanes of a wavefront, the same in every lane, without
// LDS: within each quad xor-1 and xor-2 swaps (quad_perm), then the mirror of
// each half-row of 8 and of each row of 16 (row_half_mirror, row_mirror)
// leave every lane of a row of 16 holding that row's sum; the four row sums
// are added in row order.  A fixed association, so the same bits every run.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_mov<0xb1>(v);   // quad_perm [1,0,3,2]
  v += dpp_mov<0x4e>(v);   // quad_perm [2,3,0,1]
  v += dpp_mov<0x141>(v);  // row_half_mirror
  v += dpp_mov<0x140>(v);  // row_mirror
  const int i = __builtin_bit_cast(int, v);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(i, 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(i, 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(i, 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(i, 48));
  return ((r0 + r1) + r2) + r3;
}

// NPRE: features per thread whose second-layer weights are fetched before
// the first layer's sums (registers they occupy: NPRE * 3 * AP).
template <int AP>
constexpr int tail_prefetch() { return AP <= 16 ? 2 : 1; }

template <int AP, int SP, bool V4>
__global__ __launch_bounds__(kTailThreads) void k_dqn_tail(TailArgs t) {
  constexpr int NPRE = V4 ? 0 : tail_prefetch<AP>();
  __shared__ __attribute__((aligned(16))) float hs[3 * kTailMaxF];  // the sample's first-layer outputs; the last workgroup's staging
  __shared__ __attribute__((aligned(16))) float w2s[V4 ? kTailW2Lds : 1];  // vector path: W2 of every set, as stored
  __shared__ float red[kTailThreads / 64][3 * AP];
  __shared__ float qrow[3 * AP];
  __shared__ float dqrow[AP];
  __shared__ int last;
  warm_kernargs<int(sizeof(TailArgs))>();
  const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int F = t.F, A = t.A, G = t.G, S = t.splits, B = t.B;
  // a lane's feature set is its own: pointers picked by compares, not by a
  // per-lane index into the argument arrays (a vector load of the pointer)
  auto pick = [](int g, auto p0, auto p1, auto p2) { return g == 0 ? p0 : (g == 1 ? p1 : p2); };

  // 0v. (vector path) every set's W2 in flight with the first layer's
  // loads: float4 e of the sets' blocks laid end to end (threads past the
  // last re-read it and store nothing)
  f32x4 wv[V4 ? kTailW2Loads : 1];
  const int nw4 = V4 ? G * t.fa4 : 0;
  if constexpr (V4) {
#pragma unroll
    for (int i = 0; i < kTailW2Loads; ++i) {
      const int e = min(tid + i * kTailThreads, nw4 - 1), g = t.fa4div.div(e);
      wv[i] = reinterpret_cast<const f32x4*>(pick(g, t.W2[0], t.W2[1], t.W2[2]))[e - g * t.fa4];
    }
  }

  // 0. the second layer's weights of this thread's first NPRE features in
  // every set and its bias entry (threads g * AP + a), in flight with the
  // first layer's loads
  float w2p[NPRE > 0 ? NPRE : 1][3][AP];
#pragma unroll
  for (int i = 0; i < NPRE; ++i) {
    const int n = min(tid + i * kTailThreads, F - 1);
#pragma unroll
    for (int g = 0; g < 3; ++g) {
      const float* w = t.W2[g] + long(n) * A;
#pragma unroll
      for (int a = 0; a < AP; ++a) w2p[i][g][a] = w[min(a, A - 1)];
    }
  }
  float b2v = 0.f;
  bool has_b2 = false;
  {
    const int g = min(tid / AP, 2), a = min(tid - g * AP, A - 1);
    const float* b2 = g == 0 ? t.b2[0] : (g == 1 ? t.b2[1] : t.b2[2]);
    has_b2 = b2 != nullptr;
    if (tid < 3 * AP && has_b2) b2v = b2[a];
  }
  // 1. the first layer's outputs of sample b, every feature set: item
  // k = g * F + n, kTailItems items per thread per pass, every split of an
  // item loaded in one batch (SP of them, indexes past the last split
  // re-reading it and not added)
  const int items = G * F;
  const long stride = long(B) * F;  // one split's partial tile
  if constexpr (V4) {
    // four consecutive outputs of one set per item (F % 4 == 0), the same
    // sums in the same order per output
    const int items4 = items / 4;
    for (int k0 = 0; k0 < items4; k0 += kTailItems4 * kTailThreads) {
      f32x4 v[kTailItems4][SP], bias[kTailItems4];
#pragma unroll
      for (int u = 0; u < kTailItems4; ++u) {
        const int k = 4 * min(k0 + u * kTailThreads + tid, items4 - 1);  // a clamped lane's loads are dropped
        const int g = t.fdiv.div(k), n = k - g * F;
        const f32x4* p = reinterpret_cast<const f32x4*>(t.part + (long(g) * S * B + b) * F + n);
#pragma unroll
        for (int j = 0; j < SP; ++j) v[u][j] = p[(min(j, S - 1) * stride) / 4];
        const float* bg = pick(g, t.b1[0], t.b1[1], t.b1[2]);
        bias[u] = bg ? *reinterpret_cast<const f32x4*>(bg + n) : f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int u = 0; u < kTailItems4; ++u) {
        const int k4 = k0 + u * kTailThreads + tid;
        if (k4 >= items4) break;
        const int k = 4 * k4, g = t.fdiv.div(k), n = k - g * F;
        f32x4 sum = {0.f, 0.f, 0.f, 0.f};  // split order from zero, as k_splitk_reduce sums
#pragma unroll
        for (int j = 0; j < SP; ++j)
#pragma unroll
          for (int c = 0; c < 4; ++c) sum[c] += j < S ? v[u][j][c] : 0.f;
        const f32x4* p = reinterpret_cast<const f32x4*>(t.part + (long(g) * S * B + b) * F + n);
        for (int j = SP; j < S; ++j) {
          const f32x4 w = p[(j * stride) / 4];
#pragma unroll
          for (int c = 0; c < 4; ++c) sum[c] += w[c];
        }
        f32x4 h;
#pragma unroll
        for (int c = 0; c < 4; ++c) h[c] = relu_f(sum[c] + bias[u][c]);
        *reinterpret_cast<f32x4*>(pick(g, t.h[0], t.h[1], t.h[2]) + long(b) * F + n) = h;
        *reinterpret_cast<f32x4*>(hs + k) = h;
      }
    }
#pragma unroll
    for (int i = 0; i < kTailW2Loads; ++i) {
      const int e = tid + i * kTailThreads;
      if (e < nw4) reinterpret_cast<f32x4*>(w2s)[e] = wv[i];
    }
  }
  for (int k0 = 0; k0 < (V4 ? 0 : items); k0 += kTailItems * kTailThreads) {
    if (S == 0) {
      for (int u = 0; u < kTailItems; ++u) {
        const int k = k0 + u * kTailThreads + tid;
        if (k >= items) break;
        const int g = t.fdiv.div(k), n = k - g * F;
        hs[k] = pick(g, t.h[0], t.h[1], t.h[2])[long(b) * F + n];
      }
      continue;
    }
    float v[kTailItems][SP], bias[kTailItems];
#pragma unroll
    for (int u = 0; u < kTailItems; ++u) {
      const int k = min(k0 + u * kTailThreads + tid, items - 1);  // a clamped lane's loads are dropped
      const int g = t.fdiv.div(k), n = k - g * F;
      const float* p = t.part + (long(g) * S * B + b) * F + n;
#pragma unroll
      for (int j = 0; j < SP; ++j) v[u][j] = p[min(j, S - 1) * stride];
      const float* bg = pick(g, t.b1[0], t.b1[1], t.b1[2]);
      bias[u] = bg ? bg[n] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < kTailItems; ++u) {
      const int k = k0 + u * kTailThreads + tid;
      if (k >= items) break;
      const int g = t.fdiv.div(k), n = k - g * F;
      float sum = 0.f;  // split order from zero, as k_splitk_reduce sums
#pragma unroll
      for (int j = 0; j < SP; ++j) sum += j < S ? v[u][j] : 0.f;
      const float* p = t.part + (long(g) * S * B + b) * F + n;
      for (int j = SP; j < S; ++j) sum += p[j * stride];
      const float h = relu_f(sum + bias[u]);
      pick(g, t.h[0], t.h[1], t.h[2])[long(b) * F + n] = h;
      hs[k] = h;
    }
  }
  // the sample's action row and scalars (uniform loads), in flight through
  // the next phase
  float oh[AP];
#pragma unroll
  for (int a = 0; a < AP; ++a) oh[a] = t.onehot[long(b) * A + min(a, A - 1)];
  const float reward = t.rewards[b], done = t.dones[b], discount = t.discounts[b];
  const float weight = t.weights ? t.weights[b] : 1.f;
  __syncthreads();

  // 2. q_g = h_g W2_g + b2_g: per-thread partial dot products over its
  // features in increasing order, a DPP sum over each wavefront, then the
  // wavefronts in order
  float acc[3][AP];
#pragma unroll
  for (int g = 0; g < 3; ++g)
#pragma unroll
    for (int a = 0; a < AP; ++a) acc[g][a] = 0.f;
#pragma unroll
  for (int i = 0; i < NPRE; ++i) {
    const int n = tid + i * kTailThreads;
    if (n < F) {
#pragma unroll
      for (int g = 0; g < 3; ++g) {
        const float hv = hs[g * F + n];
#pragma unroll
        for (int a = 0; a < AP; ++a) acc[g][a] = fmaf(hv, w2p[i][g][a], acc[g][a]);
      }
    }
  }
  for (int n = tid + NPRE * kTailThreads; n < F; n += kTailThreads) {
#pragma unroll
    for (int g = 0; g < 3; ++g)
      if (g < G) {
        const float hv = hs[g * F + n];
        const float* w = V4 ? w2s + (g * F + n) * A : t.W2[g] + long(n) * A;
#pragma unroll
        for (int a = 0; a < AP; ++a) acc[g][a] = fmaf(hv, w[min(a, A - 1)], acc[g][a]);
      }
  }
#pragma unroll
  for (int g = 0; g < 3; ++g)
#pragma unroll
    for (int a = 0; a < AP; ++a) {
      if (g >= G || a >= A) continue;  // uniform
      const float v = wave_sum(acc[g][a]);
      if (lane == 0) red[wave][g * AP + a] = v;
    }
  __syncthreads();
  if (tid < 3 * AP) {
    const int g = tid / AP, a = tid - g * AP;
    float v = 0.f;
    if (g < G && a < A) {
#pragma unroll
      for (int w = 0; w < kTailThreads / 64; ++w) v += red[w][tid];
      if (has_b2) v += b2v;
      t.q[g][long(b) * A + a] = v;
    }
    qrow[tid] = v;
  }
  __syncthreads();

  // 3. the DQN row of sample b, from registers
  if (tid == 0) {
    float q0[AP], qs[AP], qv[AP], dq[AP];
#pragma unroll
    for (int a = 0; a < AP; ++a) {
      q0[a] = qrow[a];
      qs[a] = qrow[AP + a];
      qv[a] = qrow[(G - 1) * AP + a];
    }
    const DqnRow r = dqn_row_r<AP>(b, A, q0, qs, qv, oh, reward, done, discount, weight, t.weights != nullptr,
                                   t.delta, 1.f / float(B), t.td_abs, t.next_act, t.td_target, dq);
#pragma unroll
    for (int a = 0; a < AP; ++a) dqrow[a] = dq[a];
    float* terms = t.loss_terms ? t.loss_terms : t.partials;
    terms[2 * b] = r.h;
    terms[2 * b + 1] = r.pred;
  }
  __syncthreads();
  if (tid < A) t.dq[long(b) * A + tid] = dqrow[tid];

  // 4. dh = dq W2_0^T through the first layer's ReLU
  float dqr[AP];
#pragma unroll
  for (int a = 0; a < AP; ++a) dqr[a] = dqrow[a];  // zero past A
#pragma unroll
  for (int i = 0; i < NPRE; ++i) {
    const int n = tid + i * kTailThreads;
    if (n < F) {
      float s = 0.f;
#pragma unroll
      for (int a = 0; a < AP; ++a) s = fmaf(dqr[a], w2p[i][0][a], s);
      t.dh[long(b) * F + n] = hs[n] > 0.f ? s : 0.f;
    }
  }
  for (int n = tid + NPRE * kTailThreads; n < F; n += kTailThreads) {
    const float* w = V4 ? w2s + n * A : t.W2[0] + long(n) * A;
    float s = 0.f;
#pragma unroll
    for (int a = 0; a < AP; ++a) s = fmaf(dqr[a], w[min(a, A - 1)], s);
    t.dh[long(b) * F + n] = hs[n] > 0.f ? s : 0.f;
  }

  // 5. the last workgroup to finish sums the batch (unless the caller does)
  if (t.loss_terms) return;
  __threadfence();  // this workgroup's rows, dq and partials, visible device-wide before the count
  __syncthreads();
  if (tid == 0) last = atomicAdd(t.counter, 1u) == unsigned(gridDim.x - 1);
  __syncthreads();
  if (!last) return;
  __threadfence();  // acquire: every workgroup's writes are visible to the loads below

  float* part = hs;                   // 2 B per-sample loss terms and predictions
  float* dqs = hs + kSyncPartials;    // a chunk of dq rows
  for (int e = tid; e < 2 * B; e += kTailThreads) part[e] = t.partials[e];

  // dW2 = h_0^T dq (when asked for), two features per thread per pass; dq
  // staged in LDS a chunk of samples at a time as [kTailChunk][AP] rows, zero
  // past the batch and past A.  A chunk's h_0 and dq loads are all issued
  // before the barrier that waits for them: one memory round trip per pass
  // and chunk.
  constexpr int DQV = (kTailChunk * AP + kTailThreads - 1) / kTailThreads;
  const float* h0 = t.h[0];
  float gb = 0.f;
  const int fw = t.dW2 ? F : 0;  // uniform: no pass when the caller forms dW2
  for (int n0 = 0; n0 < fw; n0 += 2 * kTailThreads) {  // uniform trip counts: the barriers below
    int nn[2], nc[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      nn[i] = n0 + i * kTailThreads + tid;
      nc[i] = min(nn[i], F - 1);
    }
    float gw[2][AP];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int a = 0; a < AP; ++a) gw[i][a] = 0.f;
    for (int j0 = 0; j0 < B; j0 += kTailChunk) {
      const int rows = min(kTailChunk, B - j0);
      float hv[2][kTailChunk], dqv[DQV];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < kTailChunk; ++j) hv[i][j] = h0[long(j0 + min(j, rows - 1)) * F + nc[i]];
#pragma unroll
      for (int u = 0; u < DQV; ++u) {
        const int e = u * kTailThreads + tid, j = e / AP, a = e - j * AP;
        dqv[u] = t.dq[long(j0 + min(j, rows - 1)) * A + min(a, A - 1)];
        dqv[u] = j < rows && a < A ? dqv[u] : 0.f;
      }
      __syncthreads();  // the previous chunk's readers of dqs are done
#pragma unroll
      for (int u = 0; u < DQV; ++u) {
        const int e = u * kTailThreads + tid;
        if (e < kTailChunk * AP) dqs[e] = dqv[u];
      }
      __syncthreads();
      if (n0 == 0 && tid < A)
        for (int j = 0; j < rows; ++j) gb += dqs[j * AP + tid];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < kTailChunk; ++j) hv[i][j] = j < rows ? hv[i][j] : 0.f;
#pragma unroll
      for (int j = 0; j < kTailChunk; ++j)
#pragma unroll
        for (int a = 0; a < AP; ++a) {
          const float d = dqs[j * AP + a];
          gw[0][a] = fmaf(hv[0][j], d, gw[0][a]);
          gw[1][a] = fmaf(hv[1][j], d, gw[1][a]);
        }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
      if (nn[i] < F)
#pragma unroll
        for (int a = 0; a < AP; ++a)
          if (a < A) {
            float* o = t.dW2 + long(nn[i]) * A + a;
            *o = t.beta_w != 0.f ? gw[i][a] + t.beta_w * *o : gw[i][a];
          }
  }
  if (t.db2 && tid < A) t.db2[tid] = t.beta_w != 0.f ? gb + t.beta_w * t.db2[tid] : gb;
  __syncthreads();
  if (tid == 0) {
    const float invB = 1.f / float(B);
    float sh = 0.f, sp = 0.f;
#pragma unroll 8
    for (int j = 0; j < B; ++j) {  // sample order: the same sum on every run
      sh += part[2 * j];
      sp += part[2 * j + 1];
    }
    *t.loss = sh * invB;
    if (t.mean_q) *t.mean_q = sp * invB;
    __hip_atomic_store(t.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace ttrl

using namespace ttrl;

extern "C" {

int ttrl_dqn_tail(ttrl_ctx* ctx, const ttrl_dqn_tail_desc* d) {
  TTRL_REQUIRE(ctx && d, "ttrl_dqn_tail: null argument");
  const int B = d->B, K = d->K, F = d->F, A = d->A, G = d->groups;
  TTRL_REQUIRE(G == 2 || G == 3, "ttrl_dqn_tail: 2 (vanilla) or 3 (double) feature sets, got %d", G);
  TTRL_REQUIRE(B > 0 && B <= kTailMaxB, "ttrl_dqn_tail: batch %d outside [1, %d]", B, kTailMaxB);
  TTRL_REQUIRE(K > 0 && F > 0 && F <= kTailMaxF, "ttrl_dqn_tail: %d hidden units outside [1, %d]", F, kTailMaxF);
  TTRL_REQUIRE(A > 0 && A <= kTailMaxA, "ttrl_dqn_tail: %d actions outside [1, %d]", A, kTailMaxA);
  TTRL_REQUIRE(d->delta > 0.f, "ttrl_dqn_tail: huber delta must be > 0");
  TTRL_REQUIRE(d->actions_onehot && d->rewards && d->dones && d->discounts && d->dq && d->dh,
               "ttrl_dqn_tail: null argument");
  TTRL_REQUIRE(d->dW2 || !d->db2, "ttrl_dqn_tail: a bias gradient without the weight gradient");
  TTRL_REQUIRE(d->loss || d->loss_terms, "ttrl_dqn_tail: neither loss nor loss_terms given");
  TTRL_REQUIRE(!d->loss_terms || !d->dW2,
               "ttrl_dqn_tail: with loss_terms the second layer's gradients are the caller's (dW2 must be NULL)");
  TTRL_REQUIRE(long(B) * K * 4 < kMaxOperandBytes && long(K) * F * 4 < kMaxOperandBytes,
               "ttrl_dqn_tail: an operand of 2^30 bytes or more is not supported");
  bool al = true;
  for (int g = 0; g < G; ++g) {
    TTRL_REQUIRE(d->x[g] && d->W1[g] && d->h[g] && d->W2[g] && d->q[g], "ttrl_dqn_tail: null pointer in set %d", g);
    al = al && aligned16(d->x[g]);
  }
  bool wal = true;
  for (int g = 0; g < G; ++g) wal = wal && aligned16(d->W1[g]);

  // the first layer, h = relu(x W1 + b1)
  EpStore ep;
  ep.M = B;
  ep.N = F;
  ep.ldc = F;
  ep.relu = 1;
  LdColK lb;  // B(k, n) = W1[k][n]
  lb.ld = F;
  lb.rows = F;
  lb.K = K;
  LdRowK la;  // A(m, k) = x[m][k]
  la.ld = K;
  la.rows = B;
  la.K = K;
  for (int g = 0; g < G; ++g) {
    ep.C[g] = d->h[g];
    ep.bias[g] = d->b1[g];
    lb.p[g] = d->W1[g];
    la.p[g] = d->x[g];
  }
  lb.vec_ok(wal);
  la.vec_ok(al);
  GemmPlan plan;
  int rc = run_gemm_deferred<kFc1Cfgs>(ctx, la, lb, ep, B, F, K, G, "ttrl_dqn_tail", &plan);
  if (rc) return rc;

  TailArgs t{};
  t.B = B;
  t.F = F;
  t.A = A;
  t.G = G;
  t.splits = plan.splits > 1 ? plan.splits : 0;
  t.fdiv.set(F);
  long wsf = 0;
  t.part = ctx_workspace(ctx, &wsf);
  for (int g = 0; g < 3; ++g) {
    const int s = g < G ? g : 0;
    t.h[g] = d->h[s];
    t.b1[g] = d->b1[s];
    t.W2[g] = d->W2[s];
    t.b2[g] = d->b2[s];
    t.q[g] = d->q[s];
  }
  t.onehot = d->actions_onehot;
  t.rewards = d->rewards;
  t.dones = d->dones;
  t.discounts = d->discounts;
  t.weights = d->is_weights;
  t.delta = d->delta;
  t.loss = d->loss;
  t.mean_q = d->mean_q;
  t.td_abs = d->td_abs;
  t.dq = d->dq;
  t.next_act = d->next_actions;
  t.td_target = d->td_target;
  t.dh = d->dh;
  t.dW2 = d->dW2;
  t.db2 = d->db2;
  t.beta_w = d->beta_w;
  unsigned* words = ctx_sync_words(ctx);
  t.counter = words + kSyncDqnTail;
  t.partials = reinterpret_cast<float*>(words + kSyncCounters);
  t.loss_terms = d->loss_terms;
  const int ap = A <= 8 ? 8 : (A <= 16 ? 16 : 32);
  // partials per output loaded in one batch: 8, 12 or kTailSplits (16)
  const int sp = t.splits <= 8 ? 8 : (t.splits <= 12 ? 12 : kTailSplits);
  // the vector path: split partials, biases, outputs and W2 as aligned
  // float4s, every set's W2 within the LDS stage
  bool v4 = t.splits > 0 && F % 4 == 0 && (F * A) % 4 == 0 && G * F * A <= kTailW2Lds && aligned16(t.part);
  for (int g = 0; g < G; ++g)
    v4 = v4 && aligned16(d->h[g]) && aligned16(d->W2[g]) && (!d->b1[g] || aligned16(d->b1[g]));
  t.fa4 = F * A / 4;
  t.fa4div.set(std::max(t.fa4, 1));
  auto launch = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3(unsigned(B)), dim3(kTailThreads), 0, stream_of(ctx), t);
    return check_launch("ttrl_dqn_tail");
  };
  auto by_sp = [&](auto k8, auto k12, auto k16) { return sp == 8 ? launch(k8) : (sp == 12 ? launch(k12) : launch(k16)); };
  if (v4) {
    if (ap == 8) return by_sp(k_dqn_tail<8, 8, true>, k_dqn_tail<8, 12, true>, k_dqn_tail<8, kTailSplits, true>);
    if (ap == 16) return by_sp(k_dqn_tail<16, 8, true>, k_dqn_tail<16, 12, true>, k_dqn_tail<16, kTailSplits, true>);
    return by_sp(k_dqn_tail<32, 8, true>, k_dqn_tail<32, 12, true>, k_dqn_tail<32, kTailSplits, true>);
  }
  if (ap == 8) return by_sp(k_dqn_tail<8, 8, false>, k_dqn_tail<8, 12, false>, k_dqn_tail<8, kTailSplits, false>);
  if (ap == 16) return by_sp(k_dqn_tail<16, 8, false>, k_dqn_tail<16, 12, false>, k_dqn_tail<16, kTailSplits, false>);
  return by_sp(k_dqn_tail<32, 8, false>, k_dqn_tail<32, 12, false>, k_dqn_tail<32, kTailSplits, false>);
}

}  // extern "C"
