// The SAC learner update as eight row-block launches (ttrl/algos/sac/agent.py:218-238,
// ttrl/algos/sac/losses.py:25-94, ttrl/algos/gaussian.py:55-117, ttrl/algos/sac/policy.py:30-40).
//
// Every network here is Linear(in -> H) -> ReLU -> Linear(H -> H) -> ReLU ->
// a narrow head, H a multiple of 64 up to 256.  A launch works on blocks of
// 16 rows; each workgroup owns 64 of the H columns of the one wide (H x H)
// product of its stage, so a block of rows is spread over H / 64
// workgroups.  The narrow layers either side of the wide one are row-local
// and run inside the same workgroup: the first layer (in <= 64) is formed
// straight into the LDS operand of the wide product, and the head after it
// (the Gaussian head's 2 x d columns, a critic's single column, the action
// columns of a critic's input gradient) is left as one partial dot product
// per 64-column quarter, summed in quarter order by the next stage.  The
// per-row pieces in between (the squashed sample, the soft target, the
// losses and their gradients, the sample's backward) are formed where a
// stage needs them.
//
//   stage 0  policy over [obs; next_obs]: layer 1, layer 2 (H x H), head partials
//   stage 1  the four critics of the critic region (targets on (s', a'), the
//            critics on (s, a)): a' sampled from the head partials, layer 1,
//            layer 2, Q partials
//   stage 2  soft target, twin-critic loss and its gradient, dq2 = dQ w3 [q2 > 0],
//            dq1 = dq2 W2^T [q1 > 0] for both critics
//   stage 3  the critics' weight and bias gradients: batched outer products
//            over the batch (W1: z^T dq1, W2: q1^T dq2, w3: q2^T dQ)
//   stage 4  the two (just stepped) critics on (s, a): a sampled, layers 1-2, Q partials
//   stage 5  actor loss terms, dQ to the smaller critic of each row, its
//            backward to layer 1 and partial d/da
//   stage 6  d/da summed, the sample's backward to the head, dh2, dh1 = dh2 P2^T [h1 > 0];
//            workgroup 0 also forms the actor, temperature and critic losses and
//            d alpha_loss / d log_alpha
//   stage 7  the policy's weight and bias gradients (outer products)
//
// Products run on v_mfma_f32_16x16x4f32: a wavefront owns one 16 x 16 tile.
// Lane l supplies, at step s of each 16-wide k block, A(row l % 16,
// k = 4 (l / 16) + s) and B(k = 4 (l / 16) + s, col l % 16), a permutation
// of the block both operands share, so a lane reads four consecutive k of
// an A row (one 128-bit LDS read) and of a transposed B row (one 128-bit
// global read).  Every sum runs in a fixed order, so replays are
// bit-identical.
#include "adam_dev.hpp"
#include "common.hpp"
#include "tile_gemm.hpp"

#include <cmath>

namespace ttrl {
namespace {

constexpr int kRows = 16;       // rows per workgroup
constexpr int kQ = 64;          // columns of the wide product per workgroup
constexpr int kThreads = 256;   // four wavefronts: four 16 x 16 tiles
constexpr int kMaxH = 256;
constexpr int kLda = kMaxH + 4;  // LDS row stride of the wide product's A operand
constexpr int kMaxIn = 64;       // first-layer inputs
constexpr int kXs = kMaxIn + 4;  // LDS row stride of the first layer's input rows
constexpr int kDhs = 20;         // LDS row stride of the policy head's gradient rows (2 x kMaxA <= 16 used)
constexpr int kMaxA = 8;         // action dimensions
constexpr int kMaxB = 1024;      // batch rows accepted
constexpr int kTiles = kMaxH / 64;    // first-layer column tiles per wavefront
constexpr int kBlocks = kMaxIn / 16;  // first-layer k blocks
constexpr float kLog2f = 0.69314718055994530942f;
constexpr float kLog2Pif = 1.83787706640934548356f;

__device__ __forceinline__ float relu_s(float x) { return x > 0.f ? x : 0.f; }
__device__ __forceinline__ float softplus_s(float x) { return relu_s(x) + logf(expf(-fabsf(x)) + 1.f); }
// min(a, b) as a - relu(a - b): the gradient goes to b iff a > b (ttrl/engine/ops/select.py:39-47)
__device__ __forceinline__ float min_relu_s(float a, float b) { return a - relu_s(a - b); }

// One float at byte voff + soff of a buffer resource (soff wave-uniform: it
// rides in a scalar register, so the load needs no vector address math).
__device__ __forceinline__ float ldb(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}
__device__ __forceinline__ f32x4 ldb4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

struct CriticP {
  const float *W1, *b1, *W2, *b2, *w3, *b3;
};

struct FusedArgs {
  int B, O, A, H, nq;
  const float *P1, *p1, *P2, *p2, *Wm, *bm, *Wl, *bl;
  float lo, hi;
  const float *centre, *half;
  float log_det;
  CriticP cr[4];
  const float *obs_pair, *actions, *obs_actions, *noise_pair;
  const float *rewards, *dones, *discounts, *weights;
  const float* log_alpha;
  float target_entropy;
  int learn_alpha;
  float *h1, *h2, *headp, *head, *act, *u;
  float *q1, *q2, *qp, *q1pi, *q2pi, *qppi;
  float *dQ, *dq2, *dq1, *dap, *dhead, *dh2, *dh1, *terms;
  float *critic_loss, *alpha, *actor_loss, *alpha_loss, *q_target, *td_abs, *logp;
  float* g_log_alpha;
  // the fused Adam steps' counts and hyperparameters (critic, actor,
  // temperature), whose scalars stage 0 forms into adam_sc
  int nsc;
  const int* sstep[3];
  float slr[3], sb1[3], sb2[3], seps[3];
  float* adam_sc;
};

// Each stage issues every global load it needs before its first wait:
// the loads of a workgroup then share one memory round trip, and what
// follows runs from registers and LDS.  Loads are unconditional (indices
// clamped into the operand, the value selected afterwards): a load inside
// a branch taken by some lanes only is followed by a wait where the
// branch joins.

// The wide product's B operand for this lane's column `col`: b[j] holds
// B(k, col) for k = 16 j + 4 (lane / 16) + s, s = 0..3, k < K (K a multiple
// of 16).  TRANS: B(k, n) = W[n * ldw + k], one 16-byte load per j; else
// B(k, n) = W[k * ldw + n], the row's offset in a scalar register.  W has
// `rows` rows of ldw floats.
template <bool TRANS>
__device__ __forceinline__ void load_b(const float* W, int ldw, int rows, int K, int col, f32x4 (&b)[kMaxH / 16]) {
  const int g = (threadIdx.x & 63) >> 4;
  const __amdgpu_buffer_rsrc_t res = make_res(W, uint32_t(rows) * uint32_t(ldw) * 4u);
#pragma unroll
  for (int j = 0; j < kMaxH / 16; ++j) {
    if (16 * j < K) {  // uniform
      if constexpr (TRANS) {
        b[j] = ldb4(res, (uint32_t(col) * uint32_t(ldw) + 4u * g) * 4u, 64u * j);
      } else {
        const uint32_t base = (uint32_t(4 * g) * uint32_t(ldw) + col) * 4u;
#pragma unroll
        for (int s = 0; s < 4; ++s) b[j][s] = ldb(res, base, uint32_t(16 * j + s) * uint32_t(ldw) * 4u);
      }
    }
  }
}

// acc(4 rows x 1 column per lane) = A[0:16][0:K] x B[0:K][col], A in LDS
// (row stride kLda), B as load_b left it.
__device__ __forceinline__ f32x4 rows16_mfma(const float* At, int K, const f32x4 (&b)[kMaxH / 16]) {
  const int lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < kMaxH / 16; ++j) {
    if (16 * j < K) {
      const f32x4 x = *reinterpret_cast<const f32x4*>(At + c * kLda + 16 * j + 4 * g);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.x, b[j].x, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.y, b[j].y, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.z, b[j].z, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.w, b[j].w, acc, 0, 0, 0);
    }
  }
  return acc;
}

// The first layer's weights for this lane: wavefront w owns the 16-column
// tiles w, w + 4, ... of W [J][H]; bw[i][kb][s] = W[16 kb + 4 (lane / 16) + s]
// [16 (w + 4 i) + lane % 16] (zero past J, the buffer's end), bias[i] the
// tile column's bias.
struct FirstLayerW {
  float bw[kTiles][kBlocks][4];
  float bias[kTiles];
};
__device__ __forceinline__ void load_first(const float* W, const float* b, int J, int H, FirstLayerW& f) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 4, c = lane & 15;
  const __amdgpu_buffer_rsrc_t res = make_res(W, uint32_t(J) * uint32_t(H) * 4u);
  const __amdgpu_buffer_rsrc_t rb = make_res(b, uint32_t(H) * 4u);
#pragma unroll
  for (int i = 0; i < kTiles; ++i) {
    const uint32_t col = 16u * (w + 4 * i) + c;
    f.bias[i] = 0.f;
    if (64 * i < H) f.bias[i] = ldb(rb, col * 4u, 0);  // uniform
#pragma unroll
    for (int kb = 0; kb < kBlocks; ++kb)
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        f.bw[i][kb][s] = 0.f;
        if (64 * i < H && 16 * kb < J)
          f.bw[i][kb][s] = ldb(res, (uint32_t(4 * g) * uint32_t(H) + col) * 4u, uint32_t(16 * kb + s) * uint32_t(H) * 4u);
      }
  }
}

// out[r][k] = relu(sum_j X[r][j] W[j][k] + b[k]) for the block's 16 rows and
// every k < H on the matrix cores; X in LDS (row stride kXs, zero from J up
// to the next multiple of 16).  Also stored to gout[r][k] (row stride H)
// when given.
__device__ __forceinline__ void first_layer(const float* X, int J, const FirstLayerW& f, int H, float* At,
                                            float* gout) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 4, c = lane & 15;
  f32x4 xa[kBlocks];
#pragma unroll
  for (int kb = 0; kb < kBlocks; ++kb)
    if (16 * kb < J) xa[kb] = *reinterpret_cast<const f32x4*>(X + c * kXs + 16 * kb + 4 * g);
#pragma unroll
  for (int i = 0; i < kTiles; ++i) {
    if (64 * i >= H) break;  // uniform
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < kBlocks; ++kb) {
      if (16 * kb < J) {
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[kb].x, f.bw[i][kb][0], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[kb].y, f.bw[i][kb][1], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[kb].z, f.bw[i][kb][2], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[kb].w, f.bw[i][kb][3], acc, 0, 0, 0);
      }
    }
    const int col = 16 * (w + 4 * i) + c;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 4 * g + r;
      const float v = relu_s(acc[r] + f.bias[i]);
      At[row * kLda + col] = v;
      if (gout) gout[long(row) * H + col] = v;
    }
  }
}

// A block's first-layer input rows, gathered into registers (element
// t + 256 m of the 16 x Jp slab, Jp = J rounded up to 16) and then written
// to LDS: columns [0, O) from `obs` (row stride O), [O, O + A) from
// `actions` (row stride A) unless those are sampled in the workgroup, and
// zero up to Jp.
struct InputRows {
  float v[4];
};
template <bool ACTIONS>
__device__ __forceinline__ void load_inputs(const float* obs, int O, const float* actions, int A, bool sampled,
                                            InputRows& in) {
  const int t = threadIdx.x, J = O + A, Jp = (J + 15) & ~15;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int i = t + kThreads * m, rr = i / Jp, j = i - rr * Jp, r = min(rr, kRows - 1);
    const float ov = obs[long(r) * O + min(j, O - 1)];
    float v = j < O ? ov : 0.f;
    if constexpr (ACTIONS) {
      const float av = actions[long(r) * A + min(max(j - O, 0), A - 1)];
      v = (j >= O && j < J && !sampled) ? av : v;
    }
    in.v[m] = v;
  }
}
__device__ __forceinline__ void store_inputs(const InputRows& in, int O, int A, bool sampled, float* X) {
  const int t = threadIdx.x, J = O + A, Jp = (J + 15) & ~15;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int i = t + kThreads * m, r = i / Jp, j = i - r * Jp;
    if (i < kRows * Jp && !(sampled && j >= O && j < J)) X[r * kXs + j] = in.v[m];
  }
}

// The squashed sample of policy rows prow0 .. prow0 + 15
// (ttrl/algos/gaussian.py:106-167, the stable log-density of
// ttrl/algos/sac/policy.py:30-40), one thread per (row, action dimension).
// sample_load gathers the head's quarter partials, biases, noise and
// action scale; sample_rows sums the head, clamps log_std, writes the
// action into X[row][O + j] and each dimension's two log-density terms into
// parts[row][j], [kMaxA + j]; when `store`, also the head, action and
// pre-squash u.  sample_logp adds the terms once the workgroup has
// synchronised.
struct SampleIn {
  float mp[4], lp[4], eps, bm, bl, half, centre;
};
__device__ __forceinline__ void sample_load(const FusedArgs& a, int prow0, SampleIn& s) {
  const int t = threadIdx.x, A = a.A, A2 = 2 * a.A, rows = 2 * a.B;
  const int rr = t / A, j = t - rr * A, prow = prow0 + min(rr, kRows - 1);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const long base = (long(min(q, a.nq - 1)) * rows + prow) * A2;
    s.mp[q] = a.headp[base + j];
    s.lp[q] = a.headp[base + A + j];
  }
  s.eps = a.noise_pair[long(prow) * A + j];
  s.bm = a.bm[j];
  s.bl = a.bl[j];
  s.half = a.half[j];
  s.centre = a.centre[j];
}
__device__ __forceinline__ void sample_rows(const FusedArgs& a, int prow0, const SampleIn& s, float* X, float* parts,
                                            bool store) {
  const int t = threadIdx.x, A = a.A, A2 = 2 * a.A, O = a.O;
  if (t >= kRows * A) return;
  const int row = t / A, j = t - row * A, prow = prow0 + row;
  float mu = 0.f, lsr = 0.f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    if (q < a.nq) {  // uniform
      mu += s.mp[q];
      lsr += s.lp[q];
    }
  }
  mu += s.bm;
  lsr += s.bl;
  const float ls = fminf(fmaxf(lsr, a.lo), a.hi);
  const float sigma = expf(ls);
  const float uu = mu + sigma * s.eps;
  const float z = (uu - mu) / sigma;
  parts[row * 2 * kMaxA + j] = (z * z) * -0.5f - ls;
  parts[row * 2 * kMaxA + kMaxA + j] = ((kLog2f - uu) - softplus_s(uu * -2.f)) * 2.f;
  const float act = tanhf(uu) * s.half + s.centre;
  X[row * kXs + O + j] = act;
  if (store) {
    a.head[long(prow) * A2 + j] = mu;
    a.head[long(prow) * A2 + A + j] = ls;
    a.act[long(prow) * A + j] = act;
    a.u[long(prow) * A + j] = uu;
  }
}
__device__ __forceinline__ void sample_logp(const FusedArgs& a, int prow0, const float* parts) {
  const int t = threadIdx.x;
  if (t >= kRows) return;
  float normal = 0.f, corr = 0.f;
  for (int j = 0; j < a.A; ++j) {
    normal += parts[t * 2 * kMaxA + j];
    corr += parts[t * 2 * kMaxA + kMaxA + j];
  }
  a.logp[prow0 + t] = ((normal - 0.5f * float(a.A) * kLog2Pif) - corr) - a.log_det;
}

// The 16 gate values of this thread's column t (< H) of a [rows][H] block.
__device__ __forceinline__ void load_gates(const float* src, int H, float (&gv)[kRows]) {
  const int k = threadIdx.x;
  const __amdgpu_buffer_rsrc_t res = make_res(src, uint32_t(kRows) * uint32_t(H) * 4u);
  const uint32_t kc = uint32_t(min(k, H - 1)) * 4u;
#pragma unroll
  for (int r = 0; r < kRows; ++r) gv[r] = ldb(res, kc, uint32_t(r) * uint32_t(H) * 4u);
}

// At[r][k] = gate[r][k] > 0 ? dq[r] * wk : 0 for the block's 16 rows,
// thread t column t; also stored to gout when given.
__device__ __forceinline__ void gated_rows(const float (&gv)[kRows], const float* dq, float wk, int H, float* At,
                                           float* gout) {
  const int k = threadIdx.x;
  if (k >= H) return;
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    const float v = gv[r] > 0.f ? dq[r] * wk : 0.f;
    At[r * kLda + k] = v;
    if (gout) gout[long(r) * H + k] = v;
  }
}

// The sum of x[0:n] (n <= kMaxB) in a fixed order: lane l adds x[l],
// x[l + 64], ... in turn, then the 64 lane sums are added pairwise over
// halving distances.
// Every lane of the wavefront returns the sum.
__device__ __forceinline__ float wave_sum_fixed(const float* x, int n) {
  const int lane = threadIdx.x & 63;
  float v[kMaxB / 64];
#pragma unroll
  for (int i = 0; i < kMaxB / 64; ++i) v[i] = x[min(lane + 64 * i, n - 1)];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kMaxB / 64; ++i)
    if (lane + 64 * i < n) s += v[i];
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) s += __shfl_xor(s, d, 64);
  return s;
}

// ------------------------------------------------------------ stage 0 ---
// grid (2B / 16 (+ 1), nq): the policy over [obs; next_obs].  With fused
// optimizer steps, workgroup (2B / 16, 0) forms their scalars (two
// double-precision powers each, off the stages that use them); the rest of
// that row block has nothing to do.
__global__ __launch_bounds__(kThreads) void k_sac_policy_fwd(FusedArgs a) {
  __shared__ __attribute__((aligned(16))) float X[kRows * kXs];
  __shared__ __attribute__((aligned(16))) float At[kRows * kLda];
  __shared__ float Y[kRows * (kQ + 1)];
  __shared__ float Wh[kQ * 2 * kMaxA];
  const int r0 = blockIdx.x * kRows, q = blockIdx.y, t = threadIdx.x;
  const int O = a.O, H = a.H, A = a.A, A2 = 2 * a.A, rows = 2 * a.B;
  if (r0 == rows) {  // uniform
    if (q == 0 && t < a.nsc) {
      float at, et;
      adam_scalars_at(*a.sstep[t] + 1, a.slr[t], a.sb1[t], a.sb2[t], a.seps[t], at, et);
      a.adam_sc[2 * t] = at;
      a.adam_sc[2 * t + 1] = et;
    }
    return;
  }
  const int lane = t & 63, w = t >> 6, g = lane >> 4, c = lane & 15;
  const int col = q * kQ + w * 16 + c;
  InputRows in;
  load_inputs<false>(a.obs_pair + long(r0) * O, O, nullptr, 0, false, in);
  float wh[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int i = t + kThreads * m, n = min(i / A2, kQ - 1), j = i % A2, hc = q * kQ + n;
    const float vm = a.Wm[long(hc) * A + min(j, A - 1)], vl = a.Wl[long(hc) * A + max(j - A, 0)];
    wh[m] = j < A ? vm : vl;
  }
  FirstLayerW f1;
  load_first(a.P1, a.p1, O, H, f1);
  f32x4 b[kMaxH / 16];
  load_b<false>(a.P2, H, H, H, col, b);
  const float bias = a.p2[col];
  store_inputs(in, O, 0, false, X);
#pragma unroll
  for (int m = 0; m < 4; ++m)
    if (t + kThreads * m < kQ * A2) Wh[t + kThreads * m] = wh[m];
  __syncthreads();
  first_layer(X, O, f1, H, At, q == 0 ? a.h1 + long(r0) * H : nullptr);
  __syncthreads();
  const f32x4 acc = rows16_mfma(At, H, b);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 4 * g + i;
    const float y = relu_s(acc[i] + bias);
    a.h2[long(r0 + row) * H + col] = y;
    Y[row * (kQ + 1) + w * 16 + c] = y;
  }
  __syncthreads();
  if (t < kRows * A2) {
    const int row = t / A2, j = t - row * A2;
    float s = 0.f;
    for (int n = 0; n < kQ; ++n) s = fmaf(Y[row * (kQ + 1) + n], Wh[n * A2 + j], s);
    a.headp[(long(q) * rows + r0 + row) * A2 + j] = s;
  }
}

// ------------------------------------------------------ stages 1 and 4 ---
// grid (B / 16, nq, G).  REGION 0: the critic region's four groups (0, 1:
// target critics on (next_obs, a' sampled here); 2, 3: the critics on
// (obs, the batch's actions)).  REGION 1: the actor region's two groups (the
// critics on (obs, a sampled here)).
template <int REGION>
__global__ __launch_bounds__(kThreads) void k_sac_critic_fwd(FusedArgs a) {
  __shared__ __attribute__((aligned(16))) float X[kRows * kXs];
  __shared__ __attribute__((aligned(16))) float At[kRows * kLda];
  __shared__ float Y[kRows * (kQ + 1)];
  __shared__ float W3[kQ];
  __shared__ float parts[kRows * 2 * kMaxA];
  const int r0 = blockIdx.x * kRows, q = blockIdx.y, grp = blockIdx.z, t = threadIdx.x;
  const int O = a.O, A = a.A, H = a.H, B = a.B;
  const int lane = t & 63, w = t >> 6, g = lane >> 4, c = lane & 15;
  const int col = q * kQ + w * 16 + c;
  const CriticP cp = REGION == 0 ? a.cr[grp] : a.cr[2 + grp];
  const bool next = REGION == 0 && grp < 2;        // rows of next_obs
  const bool sampled = REGION == 1 || grp < 2;      // actions sampled from the policy
  const int prow0 = next ? B + r0 : r0;             // the rows' index among the policy's 2B rows
  InputRows in;
  load_inputs<true>(a.obs_pair + long(prow0) * O, O, a.actions + long(r0) * A, A, sampled, in);
  SampleIn si;
  sample_load(a, prow0, si);
  const float w3 = cp.w3[q * kQ + min(t, kQ - 1)];
  FirstLayerW f1;
  load_first(cp.W1, cp.b1, O + A, H, f1);
  f32x4 b[kMaxH / 16];
  load_b<false>(cp.W2, H, H, H, col, b);
  const float bias = cp.b2[col];
  store_inputs(in, O, A, sampled, X);
  if (t < kQ) W3[t] = w3;
  // the first sampling group's first quarter stores the sample of its rows
  if (sampled) sample_rows(a, prow0, si, X, parts, q == 0 && grp == 0);
  __syncthreads();
  if (sampled && q == 0 && grp == 0) sample_logp(a, prow0, parts);
  float* q1 = REGION == 0 ? a.q1 : a.q1pi;
  float* q2 = REGION == 0 ? a.q2 : a.q2pi;
  float* qp = REGION == 0 ? a.qp : a.qppi;
  first_layer(X, O + A, f1, H, At, q == 0 ? q1 + (long(grp) * B + r0) * H : nullptr);
  __syncthreads();
  const f32x4 acc = rows16_mfma(At, H, b);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 4 * g + i;
    const float y = relu_s(acc[i] + bias);
    q2[(long(grp) * B + r0 + row) * H + col] = y;
    Y[row * (kQ + 1) + w * 16 + c] = y;
  }
  __syncthreads();
  if (t < kRows) {
    float s = 0.f;
    for (int n = 0; n < kQ; ++n) s = fmaf(Y[t * (kQ + 1) + n], W3[n], s);
    qp[(long(grp) * a.nq + q) * B + r0 + t] = s;
  }
}

// ------------------------------------------------------------ stage 2 ---
// The soft target and both critics' TD errors of one row
// (ttrl/algos/sac/losses.py:46-76), from Q quarter partials in quarter order.
struct CriticRow {
  float qp[4][4], b3[4], logp, reward, done, discount, weight, log_alpha;
};
__device__ __forceinline__ void critic_row_load(const FusedArgs& a, int r, CriticRow& cr) {
  const int B = a.B, nq = a.nq;
#pragma unroll
  for (int gq = 0; gq < 4; ++gq) {
#pragma unroll
    for (int q = 0; q < 4; ++q) cr.qp[gq][q] = a.qp[(long(gq) * nq + min(q, nq - 1)) * B + r];
    cr.b3[gq] = *a.cr[gq].b3;
  }
  cr.logp = a.logp[B + r];
  cr.reward = a.rewards[r];
  cr.done = a.dones[r];
  cr.discount = a.discounts[r];
  const float wv = (a.weights ? a.weights : a.rewards)[r];
  cr.weight = a.weights ? wv : 1.f;
  cr.log_alpha = *a.log_alpha;
}
__device__ __forceinline__ float q_sum(const float (&qp)[4], int nq, float b3) {
  float s = 0.f;
#pragma unroll
  for (int q = 0; q < 4; ++q)
    if (q < nq) s += qp[q];
  return s + b3;
}

// grid (B / 16, nq, 2): critic j's loss gradient and its backward to layer 1.
__global__ __launch_bounds__(kThreads) void k_sac_critic_bwd(FusedArgs a) {
  __shared__ __attribute__((aligned(16))) float At[kRows * kLda];
  __shared__ float dqs[kRows];
  const int r0 = blockIdx.x * kRows, q = blockIdx.y, j = blockIdx.z, t = threadIdx.x;
  const int H = a.H, B = a.B, nq = a.nq;
  const int lane = t & 63, w = t >> 6, g = lane >> 4, c = lane & 15;
  const int col = q * kQ + w * 16 + c;
  const CriticP cp = a.cr[2 + j];
  CriticRow cr;
  critic_row_load(a, r0 + min(t, kRows - 1), cr);
  float gv[kRows];
  load_gates(a.q2 + (long(2 + j) * B + r0) * H, H, gv);
  const float w3 = cp.w3[min(t, H - 1)];
  f32x4 b[kMaxH / 16];
  load_b<true>(cp.W2, H, H, H, col, b);
  float g1[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) g1[i] = a.q1[(long(2 + j) * B + r0 + 4 * g + i) * H + col];
  if (t < kRows) {
    const int r = r0 + t;
    const float invB = 1.f / float(B);
    const float alpha = expf(cr.log_alpha);
    const float qt0 = q_sum(cr.qp[0], nq, cr.b3[0]), qt1 = q_sum(cr.qp[1], nq, cr.b3[1]);
    const float q0 = q_sum(cr.qp[2], nq, cr.b3[2]), q1v = q_sum(cr.qp[3], nq, cr.b3[3]);
    const float soft = min_relu_s(qt0, qt1) - cr.logp * alpha;
    const float y = cr.reward + (soft * (1.f - cr.done)) * cr.discount;
    const float e0 = q0 - y, e1 = q1v - y;
    const float gs = cr.weight * (0.5f * invB) * 2.f;
    const float dq = (j == 0 ? e0 : e1) * gs;
    dqs[t] = dq;
    if (q == 0) a.dQ[long(j) * B + r] = dq;
    if (q == 0 && j == 0) {
      a.q_target[r] = y;
      if (a.td_abs) a.td_abs[r] = (fabsf(e0) + fabsf(e1)) * 0.5f;
      a.terms[2L * B + r] = a.weights ? (e0 * e0) * cr.weight : e0 * e0;
      a.terms[3L * B + r] = a.weights ? (e1 * e1) * cr.weight : e1 * e1;
      if (r == 0) *a.alpha = alpha;
    }
  }
  __syncthreads();
  // dq2 = dQ w3 [q2 > 0], the wide product's operand (stored once for the weight gradients)
  gated_rows(gv, dqs, w3, H, At, q == 0 ? a.dq2 + (long(j) * B + r0) * H : nullptr);
  __syncthreads();
  const f32x4 acc = rows16_mfma(At, H, b);
#pragma unroll
  for (int i = 0; i < 4; ++i) a.dq1[(long(j) * B + r0 + 4 * g + i) * H + col] = g1[i] > 0.f ? acc[i] : 0.f;
}

// ------------------------------------------------------------ stage 5 ---
// grid (B / 16, nq, 2): the actor loss's gradient into the smaller critic of
// each row (ttrl/algos/sac/losses.py:79-94) and critic j's backward to the
// action columns of its input, as quarter partials of d/da.
__global__ __launch_bounds__(kThreads) void k_sac_actor_bwd(FusedArgs a) {
  __shared__ __attribute__((aligned(16))) float At[kRows * kLda];
  __shared__ float Y[kRows * (kQ + 1)];
  __shared__ float W1a[kMaxA * kQ];
  __shared__ float dqs[kRows];
  const int r0 = blockIdx.x * kRows, q = blockIdx.y, j = blockIdx.z, t = threadIdx.x;
  const int H = a.H, B = a.B, nq = a.nq, O = a.O, A = a.A;
  const int lane = t & 63, w = t >> 6, g = lane >> 4, c = lane & 15;
  const int col = q * kQ + w * 16 + c;
  const CriticP cp = a.cr[2 + j];
  float qa[2][4], b3[2];
  {
    const int r = r0 + min(t, kRows - 1);
#pragma unroll
    for (int gq = 0; gq < 2; ++gq) {
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) qa[gq][qq] = a.qppi[(long(gq) * nq + min(qq, nq - 1)) * B + r];
      b3[gq] = *a.cr[2 + gq].b3;
    }
  }
  const float lp = a.logp[r0 + min(t, kRows - 1)], la = *a.log_alpha;
  float w1[2];  // the action rows of W1, this quarter's columns (A x kQ <= 512 values)
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    const int i = t + kThreads * m, aa = min(i / kQ, A - 1), n = i % kQ;
    w1[m] = cp.W1[long(O + aa) * H + q * kQ + n];
  }
  float gv[kRows];
  load_gates(a.q2pi + (long(j) * B + r0) * H, H, gv);
  const float w3 = cp.w3[min(t, H - 1)];
  f32x4 b[kMaxH / 16];
  load_b<true>(cp.W2, H, H, H, col, b);
  float g1[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) g1[i] = a.q1pi[(long(j) * B + r0 + 4 * g + i) * H + col];
#pragma unroll
  for (int m = 0; m < 2; ++m)
    if (t + kThreads * m < A * kQ) W1a[t + kThreads * m] = w1[m];
  if (t < kRows) {
    const int r = r0 + t;
    const float invB = 1.f / float(B);
    const float q0 = q_sum(qa[0], nq, b3[0]), q1v = q_sum(qa[1], nq, b3[1]);
    const bool second = q0 - q1v > 0.f;
    dqs[t] = (j == (second ? 1 : 0)) ? -invB : 0.f;
    if (q == 0 && j == 0) {
      const float alpha = expf(la);
      a.terms[r] = lp * alpha - min_relu_s(q0, q1v);
      a.terms[long(B) + r] = lp + a.target_entropy;
    }
  }
  __syncthreads();
  gated_rows(gv, dqs, w3, H, At, nullptr);
  __syncthreads();
  const f32x4 acc = rows16_mfma(At, H, b);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 4 * g + i;
    Y[row * (kQ + 1) + w * 16 + c] = g1[i] > 0.f ? acc[i] : 0.f;
  }
  __syncthreads();
  if (t < kRows * A) {
    const int row = t / A, aa = t - row * A;
    const float* w1r = W1a + aa * kQ;
    float s = 0.f;
    for (int n = 0; n < kQ; ++n) s = fmaf(Y[row * (kQ + 1) + n], w1r[n], s);
    a.dap[((long(j) * nq + q) * B + r0 + row) * A + aa] = s;
  }
}

// ------------------------------------------------------------ stage 6 ---
// grid (B / 16 + 1, nq): d/da of every row, the sample's backward to the head
// (the reparameterised path and the log-density's explicit terms), dh2 and
// dh1.  The extra row block's workgroup (B / 16, 0) forms the update's scalar
// losses and the temperature's gradient from the terms stages 2 and 5 left;
// the rest of that row block has nothing to do.
__global__ __launch_bounds__(kThreads) void k_sac_policy_bwd(FusedArgs a) {
  __shared__ __attribute__((aligned(16))) float At[kRows * kLda];
  __shared__ __attribute__((aligned(16))) float DH[kRows * kDhs];  // dhead rows, zero from 2A to 16
  __shared__ float sums[4];
  const int r0 = blockIdx.x * kRows, q = blockIdx.y, t = threadIdx.x;
  const int H = a.H, B = a.B, nq = a.nq, A = a.A, A2 = 2 * a.A;
  const float invB = 1.f / float(B);
  if (r0 == B) {  // uniform: the loss sums
    if (q != 0) return;
    const int w = t >> 6;
    const float s = wave_sum_fixed(a.terms + long(w) * B, B);
    if ((t & 63) == 0) sums[w] = s;
    __syncthreads();
    if (t == 0) {
      *a.actor_loss = sums[0] * invB;
      *a.critic_loss = (sums[2] * invB + sums[3] * invB) * 0.5f;
      if (a.learn_alpha) {
        const float la = *a.log_alpha;
        if (a.alpha_loss) *a.alpha_loss = (la * (sums[1] * invB)) * -1.f;
        if (a.g_log_alpha) *a.g_log_alpha = (sums[1] * invB) * -1.f;
      }
    }
    return;
  }
  const int lane = t & 63, w = t >> 6, g = lane >> 4, c = lane & 15;
  const int col = q * kQ + w * 16 + c;
  // per (row, action dimension): the d/da partials, head, noise, u
  float dp[2][4];
  const int prr = min(t / A, kRows - 1), paa = t % A, pr = r0 + prr;
#pragma unroll
  for (int jj = 0; jj < 2; ++jj)
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) dp[jj][qq] = a.dap[((long(jj) * nq + min(qq, nq - 1)) * B + pr) * A + paa];
  const float mu = a.head[long(pr) * A2 + paa], ls = a.head[long(pr) * A2 + A + paa];
  const float eps = a.noise_pair[long(pr) * A + paa], uu = a.u[long(pr) * A + paa];
  const float half = a.half[paa], la = *a.log_alpha;
  // dh2 on the matrix cores: B(kk, n) = Wm[n][kk] (kk < A), Wl[n][kk - A]
  // (A <= kk < 2A), zero to 16; wavefront w owns the column tiles w, w + 4, ...
  // The h2 gates in the product's layout: rows 4 g + i of each tile column.
  float wb[kTiles][4], hg[kTiles][4];
#pragma unroll
  for (int i = 0; i < kTiles; ++i) {
    const int n = min(16 * (w + 4 * i) + c, H - 1);
#pragma unroll
    for (int s2 = 0; s2 < 4; ++s2) {
      const int kk = 4 * g + s2;
      const float vm = a.Wm[long(n) * A + min(kk, A - 1)];
      const float vl = a.Wl[long(n) * A + min(max(kk - A, 0), A - 1)];
      wb[i][s2] = kk < A ? vm : (kk < 2 * A ? vl : 0.f);
      hg[i][s2] = a.h2[long(r0 + 4 * g + s2) * H + n];
    }
  }
  f32x4 b[kMaxH / 16];
  load_b<true>(a.P2, H, H, H, col, b);
  float g1[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) g1[i] = a.h1[long(r0 + 4 * g + i) * H + col];
  if (t < kRows * A) {
    const int row = t / A, aa = t - row * A, r = r0 + row;
    float ga = 0.f;
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
#pragma unroll
      for (int qq = 0; qq < 4; ++qq)
        if (qq < nq) ga += dp[jj][qq];
    const float alpha = expf(la);
    const float sigma = expf(ls);
    const float z = (uu - mu) / sigma;
    const float th = tanhf(uu);
    const float glp = alpha * invB;
    const float gu = ga * half * (1.f - th * th) + glp * (2.f * th - z / sigma);
    const float gmu = gu + glp * (z / sigma);
    float gls = gu * (sigma * eps) + glp * (z * z - 1.f);
    gls = (ls > a.lo && ls < a.hi) ? gls : 0.f;
    DH[row * kDhs + aa] = gmu;
    DH[row * kDhs + A + aa] = gls;
    if (q == 0) {
      a.dhead[long(r) * A2 + aa] = gmu;
      a.dhead[long(r) * A2 + A + aa] = gls;
    }
  }
  {
    const int zr = t >> 4, zc = t & 15;  // the zero columns of the dhead rows
    if (zc >= A2) DH[zr * kDhs + zc] = 0.f;
  }
  __syncthreads();
  // dh2 = (dhead Wh^T) [h2 > 0]
  {
    const f32x4 x = *reinterpret_cast<const f32x4*>(DH + c * kDhs + 4 * g);
#pragma unroll
    for (int i = 0; i < kTiles; ++i) {
      if (64 * i >= H) break;  // uniform
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.x, wb[i][0], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.y, wb[i][1], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.z, wb[i][2], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.w, wb[i][3], acc, 0, 0, 0);
      const int n = 16 * (w + 4 * i) + c;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 4 * g + r;
        const float v = hg[i][r] > 0.f ? acc[r] : 0.f;
        At[row * kLda + n] = v;
        if (q == 0) a.dh2[long(r0 + row) * H + n] = v;
      }
    }
  }
  __syncthreads();
  const f32x4 acc = rows16_mfma(At, H, b);
#pragma unroll
  for (int i = 0; i < 4; ++i) a.dh1[long(r0 + 4 * g + i) * H + col] = g1[i] > 0.f ? acc[i] : 0.f;
}

// --------------------------------------------------------- stages 3, 7 ---
// Weight and bias gradients as outer products over the batch:
// dw[m][n] = sum_b u[b][m] v[b][n], db[n] = sum_b v[b][n] (row M of the
// tile grid, u taken as 1).  A workgroup owns 16 rows x 64 columns of one
// problem, a wavefront one 16 x 16 tile.  The batch runs in chunks of 256
// rows: the workgroup loads its u columns and v columns of a chunk with
// coalesced loads (v 16 bytes at a time when its width allows), stages them
// in LDS and reads the products' operands from there; the next chunk's
// loads are issued before the current chunk's products.
constexpr int kMaxOuter = 8;
constexpr int kOC = 256;  // batch rows per chunk
constexpr int kUs = 20;   // LDS row strides: lanes of one operand read fall in distinct banks
constexpr int kVs = 68;
struct OuterProb {
  const float* u;
  int ldu, M;
  const float* v;
  int ldv, N;
  float* dw;
  float* db;
  int tiles_n, wg0;
  int vec;  // v read 16 bytes at a time (N and ldv multiples of 4, v 16-byte aligned); else N <= 16
  long offw, offb;  // with a fused Adam step: dw's and db's element offsets in the stepped arena
};
// A fused Adam step over one arena (the layout of ttrl_adam_range) and, when
// target is given, the Polyak blend of each stepped element into it.
struct OuterAdam {
  float *p, *S, *V;
  const float* sc;  // the step's fused scalars (alpha_t, eps_t), formed by stage 0
  float lr, b1, b2, eps, wd;
  float* partials;  // one sum of g^2 per workgroup
  float* target;
  float keep, tau;
};
struct OuterArgs {
  int nbatch, nprob;
  OuterProb p[kMaxOuter];
  int adam_on;   // the products' workgroups step `adam`
  OuterAdam adam;
  int nwg;       // the products' workgroups; workgroup nwg (when alpha_on) steps the temperature
  int alpha_on;
  OuterAdam alpha;
  long alpha_off;  // the temperature's element in its arena
  const float* alpha_g;
};

// The temperature's Adam step (one element; the finish sums one partial).
__device__ void alpha_step(const OuterArgs& a) {
  const OuterAdam& q = a.alpha;
  const long o = a.alpha_off;
  const float pv0 = q.p[o], sv0 = q.S[o], vv0 = q.V[o], g = *a.alpha_g, at = q.sc[0], et = q.sc[1];
  if (threadIdx.x == 0) {
    float pv = pv0, sv = sv0, vv = vv0, gsq = 0.f;
    adam1(pv, g, sv, vv, q.b1, q.b2, q.wd, et, at, gsq);
    q.p[o] = pv;
    q.S[o] = sv;
    q.V[o] = vv;
    q.partials[0] = gsq;
  }
}

__global__ __launch_bounds__(kThreads) void k_outer_grads(OuterArgs a) {
  __shared__ float Us[kOC * kUs];
  __shared__ __attribute__((aligned(16))) float Vs[kOC * kVs];
  __shared__ float red[kThreads / 64];
  const int wg = blockIdx.x;
  if (a.alpha_on && wg == a.nwg) {  // uniform
    alpha_step(a);
    return;
  }
  int k = 0;
#pragma unroll
  for (int i = 1; i < kMaxOuter; ++i)
    if (i < a.nprob && wg >= a.p[i].wg0) k = i;
  const OuterProb& p = a.p[k];
  const int local = wg - p.wg0, tm = local / p.tiles_n, tn = local - tm * p.tiles_n;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, g = lane >> 4, c = lane & 15;
  const int nb = a.nbatch;
  const bool vec = p.vec != 0;
  // this thread's loads: rows (t / 16) + 16 i of the chunk; u column um, v columns vc (.. vc + 3)
  const int lr = t >> 4, lc = t & 15;
  const int um = min(tm * kRows + lc, p.M - 1);
  const int vc = vec ? min(tn * kQ + 4 * lc, p.N - 4) : min(tn * kQ + lc, p.N - 1);
  // this lane's operands: A row m, B column col
  const int m = tm * kRows + c, col = tn * kQ + w * 16 + c;
  const bool mrow = m < p.M;
  const float afill = (m == p.M && p.db != nullptr) ? 1.f : 0.f;  // the bias row
  const bool live = tn * kQ + w * 16 < p.N && (vec || w == 0);  // uniform: this wavefront's tile has columns
  float uu[16];
  f32x4 vv[16];
  auto load = [&](int kb) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const long kk = min(kb + lr + 16 * i, nb - 1);
      uu[i] = p.u[kk * p.ldu + um];
      if (vec) vv[i] = *reinterpret_cast<const f32x4*>(p.v + kk * p.ldv + vc);
      else vv[i].x = p.v[kk * p.ldv + vc];
    }
  };
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  load(0);
  // the stepped elements' parameters, moments and targets, in flight with the batch
  const bool adam = a.adam_on != 0;
  long eo[4];
  bool ev[4];
  float pp[4] = {}, ps[4] = {}, pvv[4] = {}, pt[4] = {};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = tm * kRows + 4 * g + i;
    ev[i] = col < p.N && (row < p.M || (row == p.M && p.db));
    eo[i] = !ev[i] ? 0 : (row < p.M ? p.offw + long(row) * p.N + col : p.offb + col);
    if (adam) {
      pp[i] = a.adam.p[eo[i]];
      ps[i] = a.adam.S[eo[i]];
      pvv[i] = a.adam.V[eo[i]];
      if (a.adam.target) pt[i] = a.adam.target[eo[i]];
    }
  }
  const float at = adam ? a.adam.sc[0] : 0.f, et = adam ? a.adam.sc[1] : 0.f;
  for (int kb = 0; kb < nb; kb += kOC) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = lr + 16 * i;
      Us[r * kUs + lc] = uu[i];
      if (vec) *reinterpret_cast<f32x4*>(Vs + r * kVs + 4 * lc) = vv[i];
      else Vs[r * kVs + lc] = vv[i].x;
    }
    __syncthreads();
    if (kb + kOC < nb) load(kb + kOC);
    if (live) {
#pragma unroll
      for (int j = 0; j < kOC / 16; ++j) {
        if (kb + 16 * j < nb) {  // uniform
#pragma unroll
          for (int s2 = 0; s2 < 4; ++s2) {
            const int r = 16 * j + 4 * g + s2;
            const float x = Us[r * kUs + c];
            const float y = Vs[r * kVs + w * 16 + c];
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(mrow ? x : afill, y, acc, 0, 0, 0);
          }
        }
      }
    }
    __syncthreads();
  }
  float gsq = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = tm * kRows + 4 * g + i;
    if (!ev[i]) continue;
    if (row < p.M) p.dw[long(row) * p.N + col] = acc[i];
    else p.db[col] = acc[i];
    if (adam) {
      float pv = pp[i], sv = ps[i], vv = pvv[i];
      adam1(pv, acc[i], sv, vv, a.adam.b1, a.adam.b2, a.adam.wd, et, at, gsq);
      a.adam.p[eo[i]] = pv;
      a.adam.S[eo[i]] = sv;
      a.adam.V[eo[i]] = vv;
      if (a.adam.target) a.adam.target[eo[i]] = pt[i] * a.adam.keep + pv * a.adam.tau;
    }
  }
  if (adam) {
    const float tot = block_sum<kThreads>(gsq, red);
    if (threadIdx.x == 0) a.adam.partials[wg] = tot;
  }
}

bool aligned16(const void* x) { return (reinterpret_cast<uintptr_t>(x) & 15) == 0; }

int add_outer(OuterArgs& o, int& wgs, const float* u, int ldu, int M, const float* v, int ldv, int N, float* dw,
              float* db, const char* name) {
  TTRL_REQUIRE(o.nprob < kMaxOuter, "%s: too many gradient products", name);
  TTRL_REQUIRE(u && v && dw && M > 0 && N > 0 && ldu >= M && ldv >= N, "%s: bad gradient product", name);
  OuterProb& p = o.p[o.nprob++];
  p.u = u;
  p.ldu = ldu;
  p.M = M;
  p.v = v;
  p.ldv = ldv;
  p.N = N;
  p.dw = dw;
  p.db = db;
  p.tiles_n = int(ceil_div(N, kQ));
  p.wg0 = wgs;
  p.vec = (N % 4 == 0 && ldv % 4 == 0 && aligned16(v)) ? 1 : 0;
  TTRL_REQUIRE(p.vec || N <= 16, "%s: a gradient product of width %d must have a width and row stride that are "
               "multiples of 4 and a 16-byte aligned operand", name, N);
  p.offw = p.offb = 0;
  wgs += int(ceil_div(M + (db ? 1 : 0), kRows)) * p.tiles_n;
  return TTRL_OK;
}

// The gradient products of stage 3 (the trained critics' W1, b1, W2, b2,
// w3, b3) or stage 7 (the policy's P1, p1, P2, p2, Wm, bm, Wl, bl).
int outer_problems(const ttrl_sac_fused_desc* d, int stage, OuterArgs& o, int& wgs, const char* name) {
  const int B = d->B, O = d->O, A = d->A, H = d->H;
  o.nbatch = B;
  wgs = 0;
  int rc = 0;
  if (stage == 3) {
    for (int j = 0; j < 2; ++j) {
      float* const* gc = d->g_critic[j];
      TTRL_REQUIRE(gc[0] && gc[1] && gc[2] && gc[3] && gc[4] && gc[5] && d->obs_actions && d->dq1 && d->q1 &&
                       d->dq2 && d->q2 && d->dQ,
                   "%s: stage 3: null gradient or operand", name);
      rc = add_outer(o, wgs, d->obs_actions, O + A, O + A, d->dq1 + long(j) * B * H, H, H, gc[0], gc[1], name);
      if (!rc)
        rc = add_outer(o, wgs, d->q1 + long(2 + j) * B * H, H, H, d->dq2 + long(j) * B * H, H, H, gc[2], gc[3], name);
      if (!rc) rc = add_outer(o, wgs, d->q2 + long(2 + j) * B * H, H, H, d->dQ + long(j) * B, 1, 1, gc[4], gc[5], name);
      if (rc) return rc;
    }
  } else {
    TTRL_REQUIRE(d->gP1 && d->gp1 && d->gP2 && d->gp2 && d->gWm && d->gbm && d->gWl && d->gbl && d->obs_pair &&
                     d->dh1 && d->h1 && d->dh2 && d->h2 && d->dhead,
                 "%s: stage 7: null gradient or operand", name);
    rc = add_outer(o, wgs, d->obs_pair, O, O, d->dh1, H, H, d->gP1, d->gp1, name);
    if (!rc) rc = add_outer(o, wgs, d->h1, H, H, d->dh2, H, H, d->gP2, d->gp2, name);
    if (!rc) rc = add_outer(o, wgs, d->h2, H, H, d->dhead, 2 * A, A, d->gWm, d->gbm, name);
    if (!rc) rc = add_outer(o, wgs, d->h2, H, H, d->dhead + A, 2 * A, A, d->gWl, d->gbl, name);
  }
  return rc;
}

// A fused Adam step from its range: the hyperparameters checked as
// ttrl_adam_step checks them, the partials in the range's context slot.
int outer_adam(ttrl_ctx* ctx, const ttrl_adam_range& r, OuterAdam& q, const char* name, const char* which) {
  TTRL_REQUIRE(r.p && r.g && r.m_s && r.v_s && r.step && r.n > 0, "%s: %s: null buffer or empty range", name, which);
  TTRL_REQUIRE(r.lr > 0.f && r.beta1 >= 0.f && r.beta1 < 1.f && r.beta2 >= 0.f && r.beta2 < 1.f && r.eps > 0.f &&
                   r.weight_decay >= 0.f,
               "%s: %s: bad hyperparameters", name, which);
  TTRL_REQUIRE(r.slot >= 0 && r.slot < kAdamSlots, "%s: %s: slot %d outside [0, %d)", name, which, r.slot,
               kAdamSlots);
  q = OuterAdam{r.p, r.m_s, r.v_s, nullptr, r.lr, r.beta1, r.beta2, r.eps, r.weight_decay,
                ctx_adam_partials(ctx) + long(r.slot) * kAdamSlotFloats, nullptr, 0.f, 0.f};
  return TTRL_OK;
}

// Each product's dw and db as element offsets in the stepped arena [g, g + n).
int outer_offsets(OuterArgs& o, const ttrl_adam_range& r, const char* name) {
  for (int i = 0; i < o.nprob; ++i) {
    OuterProb& p = o.p[i];
    const long ow = long(p.dw - r.g), ob = p.db ? long(p.db - r.g) : 0;
    TTRL_REQUIRE(ow >= 0 && ow + long(p.M) * p.N <= r.n && (!p.db || (ob >= 0 && ob + p.N <= r.n)),
                 "%s: gradient product %d lies outside the stepped arena", name, i);
    p.offw = ow;
    p.offb = ob;
  }
  return TTRL_OK;
}

}  // namespace
}  // namespace ttrl

using namespace ttrl;

extern "C" {

int ttrl_sac_fused_stage(ttrl_ctx* ctx, int stage, const ttrl_sac_fused_desc* d) {
  TTRL_REQUIRE(ctx && d, "ttrl_sac_fused_stage: null argument");
  const int B = d->B, O = d->O, A = d->A, H = d->H;
  TTRL_REQUIRE(B > 0 && B % kRows == 0 && B <= kMaxB, "ttrl_sac_fused_stage: batch %d must be a multiple of %d, "
               "at most %d", B, kRows, kMaxB);
  TTRL_REQUIRE(H > 0 && H % kQ == 0 && H <= kMaxH, "ttrl_sac_fused_stage: hidden width %d must be a multiple of "
               "%d, at most %d", H, kQ, kMaxH);
  TTRL_REQUIRE(A > 0 && A <= kMaxA && O > 0 && O + A <= kMaxIn, "ttrl_sac_fused_stage: %d observation and %d "
               "action dimensions (at most %d actions, %d together)", O, A, kMaxA, kMaxIn);
  TTRL_REQUIRE(aligned16(d->P2) && aligned16(d->critic[2].W2) && aligned16(d->critic[3].W2),
               "ttrl_sac_fused_stage: the H x H weights must be 16-byte aligned");
  FusedArgs a{};
  a.B = B;
  a.O = O;
  a.A = A;
  a.H = H;
  a.nq = H / kQ;
  a.P1 = d->P1;
  a.p1 = d->p1;
  a.P2 = d->P2;
  a.p2 = d->p2;
  a.Wm = d->Wm;
  a.bm = d->bm;
  a.Wl = d->Wl;
  a.bl = d->bl;
  a.lo = d->log_std_min;
  a.hi = d->log_std_max;
  a.centre = d->centre;
  a.half = d->half_width;
  a.log_det = d->log_det;
  for (int i = 0; i < 4; ++i) {
    const ttrl_sac_critic_params& c = d->critic[i];
    TTRL_REQUIRE(c.W1 && c.b1 && c.W2 && c.b2 && c.w3 && c.b3, "ttrl_sac_fused_stage: critic %d: null weight", i);
    a.cr[i] = CriticP{c.W1, c.b1, c.W2, c.b2, c.w3, c.b3};
  }
  a.obs_pair = d->obs_pair;
  a.actions = d->actions;
  a.obs_actions = d->obs_actions;
  a.noise_pair = d->noise_pair;
  a.rewards = d->rewards;
  a.dones = d->dones;
  a.discounts = d->discounts;
  a.weights = d->is_weights;
  a.log_alpha = d->log_alpha;
  a.target_entropy = d->target_entropy;
  a.learn_alpha = d->learn_alpha;
  a.h1 = d->h1;
  a.h2 = d->h2;
  a.headp = d->headp;
  a.head = d->head;
  a.act = d->act;
  a.u = d->u;
  a.q1 = d->q1;
  a.q2 = d->q2;
  a.qp = d->qp;
  a.q1pi = d->q1pi;
  a.q2pi = d->q2pi;
  a.qppi = d->qppi;
  a.dQ = d->dQ;
  a.dq2 = d->dq2;
  a.dq1 = d->dq1;
  a.dap = d->dap;
  a.dhead = d->dhead;
  a.dh2 = d->dh2;
  a.dh1 = d->dh1;
  a.terms = d->terms;
  a.critic_loss = d->critic_loss;
  a.alpha = d->alpha;
  a.actor_loss = d->actor_loss;
  a.alpha_loss = d->alpha_loss;
  a.q_target = d->q_target;
  a.td_abs = d->td_abs;
  a.logp = d->logp;
  a.g_log_alpha = d->g_log_alpha;
  const unsigned nq = unsigned(a.nq), rb = unsigned(B / kRows);
  hipStream_t st = stream_of(ctx);
  const char* name = "ttrl_sac_fused_stage";
  switch (stage) {
    case 0:
      TTRL_REQUIRE(a.P1 && a.p1 && a.P2 && a.p2 && a.Wm && a.bm && a.Wl && a.bl && a.obs_pair && a.h1 && a.h2 &&
                       a.headp,
                   "%s: stage 0: null argument", name);
      if (d->fuse_adam) {
        const ttrl_adam_range* rs[3] = {&d->critic_adam, &d->actor_adam, &d->alpha_adam};
        a.nsc = d->learn_alpha ? 3 : 2;
        for (int i = 0; i < a.nsc; ++i) {
          TTRL_REQUIRE(rs[i]->step, "%s: stage 0: a fused optimizer step without its update count", name);
          a.sstep[i] = rs[i]->step;
          a.slr[i] = rs[i]->lr;
          a.sb1[i] = rs[i]->beta1;
          a.sb2[i] = rs[i]->beta2;
          a.seps[i] = rs[i]->eps;
        }
        TTRL_REQUIRE(d->adam_scalars, "%s: fused optimizer steps need adam_scalars", name);
        a.adam_sc = d->adam_scalars;
      }
      hipLaunchKernelGGL(k_sac_policy_fwd, dim3(2 * rb + (a.nsc > 0 ? 1 : 0), nq), dim3(kThreads), 0, st, a);
      break;
    case 1:
    case 4:
      TTRL_REQUIRE(a.obs_pair && a.actions && a.noise_pair && a.headp && a.head && a.act && a.u && a.logp &&
                       a.centre && a.half,
                   "%s: stage %d: null argument", name, stage);
      if (stage == 1) {
        TTRL_REQUIRE(a.q1 && a.q2 && a.qp, "%s: stage 1: null argument", name);
        hipLaunchKernelGGL(k_sac_critic_fwd<0>, dim3(rb, nq, 4), dim3(kThreads), 0, st, a);
      } else {
        TTRL_REQUIRE(a.q1pi && a.q2pi && a.qppi, "%s: stage 4: null argument", name);
        hipLaunchKernelGGL(k_sac_critic_fwd<1>, dim3(rb, nq, 2), dim3(kThreads), 0, st, a);
      }
      break;
    case 2:
      TTRL_REQUIRE(a.qp && a.q1 && a.q2 && a.logp && a.rewards && a.dones && a.discounts && a.log_alpha && a.dQ &&
                       a.dq2 && a.dq1 && a.terms && a.q_target && a.alpha,
                   "%s: stage 2: null argument", name);
      hipLaunchKernelGGL(k_sac_critic_bwd, dim3(rb, nq, 2), dim3(kThreads), 0, st, a);
      break;
    case 5:
      TTRL_REQUIRE(a.qppi && a.q1pi && a.q2pi && a.logp && a.log_alpha && a.dap && a.terms,
                   "%s: stage 5: null argument", name);
      hipLaunchKernelGGL(k_sac_actor_bwd, dim3(rb, nq, 2), dim3(kThreads), 0, st, a);
      break;
    case 6:
      TTRL_REQUIRE(a.dap && a.head && a.noise_pair && a.u && a.h1 && a.h2 && a.dhead && a.dh2 && a.dh1 &&
                       a.terms && a.log_alpha && a.actor_loss && a.critic_loss && a.half && a.Wm && a.Wl && a.P2,
                   "%s: stage 6: null argument", name);
      hipLaunchKernelGGL(k_sac_policy_bwd, dim3(rb + 1, nq), dim3(kThreads), 0, st, a);
      break;
    case 3:
    case 7: {
      OuterArgs o{};
      int wgs = 0;
      int rc = outer_problems(d, stage, o, wgs, name);
      if (rc) return rc;
      o.nwg = wgs;
      if (d->fuse_adam) {
        const ttrl_adam_range& r = stage == 3 ? d->critic_adam : d->actor_adam;
        rc = outer_adam(ctx, r, o.adam, name, stage == 3 ? "critic_adam" : "actor_adam");
        if (!rc) rc = outer_offsets(o, r, name);
        if (rc) return rc;
        TTRL_REQUIRE(d->adam_scalars, "%s: fused optimizer steps need adam_scalars", name);
        o.adam.sc = d->adam_scalars + (stage == 3 ? 0 : 2);
        TTRL_REQUIRE(wgs <= kAdamSlotFloats, "%s: %d partial sums exceed a slot", name, wgs);
        o.adam_on = 1;
        if (stage == 3) {
          TTRL_REQUIRE(d->polyak_dst && d->tau >= 0.f && d->tau <= 1.f, "%s: stage 3: null Polyak target or tau "
                       "outside [0, 1]", name);
          o.adam.target = d->polyak_dst;
          o.adam.keep = 1.f - d->tau;
          o.adam.tau = d->tau;
        } else if (d->learn_alpha) {
          const ttrl_adam_range& ra = d->alpha_adam;
          rc = outer_adam(ctx, ra, o.alpha, name, "alpha_adam");
          if (rc) return rc;
          o.alpha.sc = d->adam_scalars + 4;
          TTRL_REQUIRE(ra.slot != r.slot, "%s: the temperature and the policy share slot %d", name, r.slot);
          const long off = d->g_log_alpha ? long(d->g_log_alpha - ra.g) : -1;
          TTRL_REQUIRE(off >= 0 && off < ra.n, "%s: g_log_alpha lies outside the temperature's arena", name);
          o.alpha_on = 1;
          o.alpha_off = off;
          o.alpha_g = d->g_log_alpha;
        }
      }
      hipLaunchKernelGGL(k_outer_grads, dim3(unsigned(wgs + o.alpha_on)), dim3(kThreads), 0, st, o);
      break;
    }
    default:
      return set_error(TTRL_EINVAL, "%s: stage %d outside [0, 7]", name, stage);
  }
  return check_launch(name);
}

int ttrl_sac_fused_adam_parts(const ttrl_sac_fused_desc* d, int stage, int* parts) {
  TTRL_REQUIRE(d && parts, "ttrl_sac_fused_adam_parts: null argument");
  TTRL_REQUIRE(stage == 3 || stage == 7, "ttrl_sac_fused_adam_parts: stage %d steps no optimizer (3 or 7)", stage);
  OuterArgs o{};
  int wgs = 0;
  const int rc = outer_problems(d, stage, o, wgs, "ttrl_sac_fused_adam_parts");
  if (rc) return rc;
  *parts = wgs;
  return TTRL_OK;
}

}  // extern "C"
